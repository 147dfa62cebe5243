// exl3_kernels.hip -- gfx950 kernels of the EXL3 packed-weight linear layer.
//
//   gemv_kernel      rows 1..32: each lane decodes 16 trellis positions of a tile
//                    straight into an fp16 MFMA A-fragment (W^T), the activations
//                    H128(x*su) arrive pre-split into fp16 hi/lo halves in the 16
//                    MFMA columns, v_mfma_f32_16x16x32_f16 accumulates in fp32;
//                    split-K partials are reduced in fixed order by the last
//                    workgroup of each 128-column group, which applies H128 and sv.
//   gemm_xprep_kernel, gemm_kernel, gemm_reduce_kernel
//                    rows > 32: H128(x*su) once in fp16 MFMA-fragment order; a
//                    workgroup (k split, column group, m-tile) decodes record kb + 1
//                    into LDS (fp16, swizzled) while v_mfma_f32_32x32x16_f16 runs on
//                    record kb, fp32 accumulation; split partials are summed in
//                    fixed order by the reduce kernel, which applies H128 and sv.
//   decode_kernel    trellis tiles -> row-major fp16, bit-exact (exl3::decode_inner).
//   reconstruct_kernel original-basis weights, bit-exact (exl3::reconstruct).
//   get_rows_kernel    GET_ROWS: columns of the original-basis weights (ggml_exl3_get_rows).
// Reference semantics: src/exl3_codec.cpp, src/exl3-ggml.cpp:51-92.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <stdint.h>

#include <type_traits>

#include "exl3_device.hpp"
#include "exl3_launch.hpp"

using namespace exl3dev;

namespace exl3k {

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
// write-back or invalidate of unrelated lines); the writer waits for its stores
// to complete before the arrival counter is bumped.
__device__ __forceinline__ void store_coherent(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// returns true in every thread of the last of `total` arriving workgroups
__device__ __forceinline__ bool arrive_last(unsigned *counter, unsigned total, int *flag_lds) {
    wait_stores();
    __syncthreads();
    if (threadIdx.x == 0)
        *flag_lds = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == total - 1;
    __syncthreads();
    return *flag_lds != 0;
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

// ============================================================== codebook
template <int CB>
__global__ void codebook_kernel(const uint16_t *__restrict__ states, size_t count, uint16_t *__restrict__ out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) out[i] = codebook_one<CB>(states[i]);
}

hipError_t launch_codebook(const uint16_t *states, size_t count, int cb, uint16_t *out, hipStream_t stream) {
    const dim3 grid((unsigned)((count + 255) / 256)), block(256);
    switch (cb) {
    case 0: codebook_kernel<0><<<grid, block, 0, stream>>>(states, count, out); break;
    case 1: codebook_kernel<1><<<grid, block, 0, stream>>>(states, count, out); break;
    default: codebook_kernel<2><<<grid, block, 0, stream>>>(states, count, out); break;
    }
    return hipGetLastError();
}

// ============================================================== H128
__global__ __launch_bounds__(64) void hadamard_kernel(float *__restrict__ values) {
    __shared__ float v[128];
    float *blk = values + (size_t)blockIdx.x * 128;
    const int t = threadIdx.x;
    v[t] = blk[t];
    v[t + 64] = blk[t + 64];
    __syncthreads();
    h128_lds(v, 1, 128, t, 64);
    blk[t] = v[t];
    blk[t + 64] = v[t + 64];
}

hipError_t launch_hadamard(float *values, size_t count, hipStream_t stream) {
    if (count) hadamard_kernel<<<dim3((unsigned)(count / 128)), dim3(64), 0, stream>>>(values);
    return hipGetLastError();
}

// ============================================================== zero fill
__global__ void zero_kernel(uint32_t *__restrict__ p, size_t words) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < words; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

hipError_t launch_zero(void *ptr, size_t bytes, hipStream_t stream) {
    const size_t words = bytes / 4;
    if (words) {
        const unsigned blocks = (unsigned)((words + 255) / 256 < 4096 ? (words + 255) / 256 : 4096);
        zero_kernel<<<dim3(blocks), dim3(256), 0, stream>>>((uint32_t *)ptr, words);
    }
    return hipGetLastError();
}

// ============================================================== decode
// One workgroup block: one 16-row tile row rk, 16 consecutive tile columns
// starting at tile bx * 16 of the slice.  Lane (wave w, lane l): tile w*4 + l/16,
// run c = l%8, h = (l%16)/8.
constexpr int kDecodePitch = 16 * 16 + 8;
template <int K, int CB>
__device__ __forceinline__ void decode_block(const uint8_t *__restrict__ src, int records_layout, size_t k, size_t n,
                                             size_t first_tile, size_t tile_count, uint16_t *__restrict__ out,
                                             size_t bx, size_t rk, uint16_t *tb) {
    constexpr int PITCH = kDecodePitch;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t t0 = bx * 16;  // first tile (relative to first_tile) of this workgroup
    const int tl = wave * 4 + (lane >> 4);
    const int c = lane & 7, h = (lane >> 3) & 1;
    if (t0 + tl < tile_count) {
        const uint32_t *tile = tile_ptr<K>(src, records_layout, k, n, rk, first_tile + t0 + tl);
        uint32_t w[RunGeo<K>::NW];
        load_run_words<K>(tile, c, h, w);
        u4 a1, a2;
        decode_run<K, CB>(w, a1, a2);
        const uint32_t p1[4] = {a1.x, a1.y, a1.z, a1.w}, p2[4] = {a2.x, a2.y, a2.z, a2.w};
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int r0 = run_slot_row(h, 2 * v), r1 = run_slot_row(h, 2 * v + 1);
            tb[r0 * PITCH + tl * 16 + c] = (uint16_t)(p1[v] & 0xffffu);
            tb[r1 * PITCH + tl * 16 + c] = (uint16_t)(p1[v] >> 16);
            tb[r0 * PITCH + tl * 16 + c + 8] = (uint16_t)(p2[v] & 0xffffu);
            tb[r1 * PITCH + tl * 16 + c + 8] = (uint16_t)(p2[v] >> 16);
        }
    }
    __syncthreads();
    const size_t count = tile_count * 16;  // output row length
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int ch = tid + 256 * i;      // 16 rows x 32 chunks of 8 halves
        const int row = ch >> 5, col8 = ch & 31;
        const int tl2 = col8 >> 1;
        if (t0 + tl2 < tile_count) {
            const u4 v = *(const u4 *)(tb + row * PITCH + col8 * 8);
            // streaming store: the fp16 output is written once and not read back here
            __builtin_nontemporal_store(v, (u4 *)(out + (rk * 16 + row) * count + (t0 + tl2) * 16 + (col8 & 1) * 8));
        }
    }
}

template <int K, int CB>
__global__ __launch_bounds__(256) void decode_kernel(const uint8_t *__restrict__ src, int records_layout, size_t k,
                                                     size_t n, size_t first_tile, size_t tile_count,
                                                     uint16_t *__restrict__ out) {
    __shared__ uint16_t tb[16 * kDecodePitch];
    decode_block<K, CB>(src, records_layout, k, n, first_tile, tile_count, out, blockIdx.x, blockIdx.y, tb);
}

// Several whole matrices of one rate in one launch: workgroup w belongs to the
// matrix m whose range [wg_begin[m], wg_begin[m + 1]) holds it, and decodes its
// block (bx, rk) = (local % gx, local / gx) with gx = ceil(n / 256).
template <int K, int CB>
__global__ __launch_bounds__(256) void decode_batch_kernel(DecodeBatch batch, int records_layout) {
    __shared__ uint16_t tb[16 * kDecodePitch];
    const unsigned w = blockIdx.x;
    int m = 0;
    for (int i = 1; i < batch.count; ++i)
        if (w >= batch.wg_begin[i]) m = i;
    const size_t k = batch.k[m], n = batch.n[m];
    const size_t gx = (n / 16 + 15) / 16, local = w - batch.wg_begin[m];
    decode_block<K, CB>((const uint8_t *)batch.src[m], records_layout, k, n, 0, n / 16, batch.out[m], local % gx,
                        local / gx, tb);
}

template <int K>
static hipError_t launch_decode_k(const void *src, int rl, int cb, size_t k, size_t n, size_t first, size_t count,
                                  uint16_t *out, hipStream_t stream) {
    const size_t tiles = count / 16;
    const dim3 grid((unsigned)((tiles + 15) / 16), (unsigned)(k / 16)), block(256);
    const uint8_t *s = (const uint8_t *)src;
    switch (cb) {
    case 0: decode_kernel<K, 0><<<grid, block, 0, stream>>>(s, rl, k, n, first / 16, tiles, out); break;
    case 1: decode_kernel<K, 1><<<grid, block, 0, stream>>>(s, rl, k, n, first / 16, tiles, out); break;
    default: decode_kernel<K, 2><<<grid, block, 0, stream>>>(s, rl, k, n, first / 16, tiles, out); break;
    }
    return hipGetLastError();
}

template <int K>
static hipError_t launch_decode_batch_k(const DecodeBatch &b, int rl, int cb, unsigned wgs, hipStream_t stream) {
    switch (cb) {
    case 0: decode_batch_kernel<K, 0><<<dim3(wgs), dim3(256), 0, stream>>>(b, rl); break;
    case 1: decode_batch_kernel<K, 1><<<dim3(wgs), dim3(256), 0, stream>>>(b, rl); break;
    default: decode_batch_kernel<K, 2><<<dim3(wgs), dim3(256), 0, stream>>>(b, rl); break;
    }
    return hipGetLastError();
}

hipError_t launch_decode_batch(const DecodeBatch &b, int rl, int bits, int cb, unsigned wgs, hipStream_t stream) {
    switch (bits) {
    case 1: return launch_decode_batch_k<1>(b, rl, cb, wgs, stream);
    case 2: return launch_decode_batch_k<2>(b, rl, cb, wgs, stream);
    case 3: return launch_decode_batch_k<3>(b, rl, cb, wgs, stream);
    case 4: return launch_decode_batch_k<4>(b, rl, cb, wgs, stream);
    case 5: return launch_decode_batch_k<5>(b, rl, cb, wgs, stream);
    case 6: return launch_decode_batch_k<6>(b, rl, cb, wgs, stream);
    case 7: return launch_decode_batch_k<7>(b, rl, cb, wgs, stream);
    default: return launch_decode_batch_k<8>(b, rl, cb, wgs, stream);
    }
}

hipError_t launch_decode(const void *src, int rl, int bits, int cb, size_t k, size_t n, size_t first, size_t count,
                         uint16_t *out, hipStream_t stream) {
    switch (bits) {
    case 1: return launch_decode_k<1>(src, rl, cb, k, n, first, count, out, stream);
    case 2: return launch_decode_k<2>(src, rl, cb, k, n, first, count, out, stream);
    case 3: return launch_decode_k<3>(src, rl, cb, k, n, first, count, out, stream);
    case 4: return launch_decode_k<4>(src, rl, cb, k, n, first, count, out, stream);
    case 5: return launch_decode_k<5>(src, rl, cb, k, n, first, count, out, stream);
    case 6: return launch_decode_k<6>(src, rl, cb, k, n, first, count, out, stream);
    case 7: return launch_decode_k<7>(src, rl, cb, k, n, first, count, out, stream);
    default: return launch_decode_k<8>(src, rl, cb, k, n, first, count, out, stream);
    }
}

// ============================================================== reconstruct
// One workgroup per 128x128 block: decode into LDS (fp32), H128 along each row
// (over n), then along each column (over k), then fp16((w * su) * sv) -- the
// operation order of src/exl3_codec.cpp:184-202, so the result is bit-exact.
template <int K, int CB>
__global__ __launch_bounds__(256) void reconstruct_kernel(const uint8_t *__restrict__ src, int records_layout,
                                                          const uint16_t *__restrict__ su,
                                                          const uint16_t *__restrict__ sv, size_t k, size_t n,
                                                          size_t first_column, size_t count,
                                                          uint16_t *__restrict__ out) {
    constexpr int P = 129;
    __shared__ float blk[128 * P];
    const int tid = threadIdx.x;
    const size_t bc = blockIdx.x, brk = blockIdx.y;  // column block (within the slice), row block
    const size_t cn0 = first_column / 16 + bc * 8, rk0 = brk * 8;
#pragma unroll 1
    for (int i = 0; i < 4; ++i) {
        const int run = tid + 256 * i;
        const int tile = run >> 4, rc = run & 15;
        const int c = rc & 7, h = rc >> 3, tr = tile >> 3, tc = tile & 7;
        const uint32_t *tp = tile_ptr<K>(src, records_layout, k, n, rk0 + tr, cn0 + tc);
        uint32_t w[RunGeo<K>::NW];
        load_run_words<K>(tp, c, h, w);
        u4 a1, a2;
        decode_run<K, CB>(w, a1, a2);
        const uint32_t p1[4] = {a1.x, a1.y, a1.z, a1.w}, p2[4] = {a2.x, a2.y, a2.z, a2.w};
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int r0 = tr * 16 + run_slot_row(h, 2 * v), r1 = tr * 16 + run_slot_row(h, 2 * v + 1);
            const int cc = tc * 16 + c;
            blk[r0 * P + cc] = half_bits_to_float((uint16_t)(p1[v] & 0xffffu));
            blk[r1 * P + cc] = half_bits_to_float((uint16_t)(p1[v] >> 16));
            blk[r0 * P + cc + 8] = half_bits_to_float((uint16_t)(p2[v] & 0xffffu));
            blk[r1 * P + cc + 8] = half_bits_to_float((uint16_t)(p2[v] >> 16));
        }
    }
    __syncthreads();
    // H128 along n for each row, one thread per row, stage order of the reference
    if (tid < 128) {
        float *v = blk + tid * P;
        for (int step = 1; step < 128; step <<= 1)
            for (int b = 0; b < 64; ++b) {
                const int i = ((b & ~(step - 1)) << 1) | (b & (step - 1));
                const float a = v[i], c2 = v[i + step];
                v[i] = a + c2;
                v[i + step] = a - c2;
            }
        for (int i = 0; i < 128; ++i) v[i] *= 0.08838834764831844055f;
    }
    __syncthreads();
    if (tid < 128) {
        float *v = blk + tid;
        for (int step = 1; step < 128; step <<= 1)
            for (int b = 0; b < 64; ++b) {
                const int i = ((b & ~(step - 1)) << 1) | (b & (step - 1));
                const float a = v[i * P], c2 = v[(i + step) * P];
                v[i * P] = a + c2;
                v[(i + step) * P] = a - c2;
            }
        for (int i = 0; i < 128; ++i) v[i * P] *= 0.08838834764831844055f;
    }
    __syncthreads();
    const size_t gcol0 = first_column + bc * 128;  // absolute column of this block
    const uint8_t *rec = records_layout ? src + ((gcol0 >> 7) * (k >> 7) + brk) * group_bytes(K) : nullptr;
    const uint16_t *su_b = records_layout ? (const uint16_t *)(rec + 2048 * K) : su + brk * 128;
    const uint16_t *sv_b = records_layout ? (const uint16_t *)(rec + 2048 * K + 256) : sv + gcol0;
    for (int e = tid; e < 128 * 128; e += 256) {
        const int row = e >> 7, col = e & 127;
        const float scaled = mul_rn_f32(blk[row * P + col], half_bits_to_float(su_b[row]));
        out[(brk * 128 + row) * count + bc * 128 + col] = float_to_half_bits(mul_rn_f32(scaled, half_bits_to_float(sv_b[col])));
    }
}

template <int K>
static hipError_t launch_reconstruct_k(const void *src, int rl, const uint16_t *su, const uint16_t *sv, int cb,
                                       size_t k, size_t n, size_t first, size_t count, uint16_t *out,
                                       hipStream_t stream) {
    const dim3 grid((unsigned)(count / 128), (unsigned)(k / 128)), block(256);
    const uint8_t *s = (const uint8_t *)src;
    switch (cb) {
    case 0: reconstruct_kernel<K, 0><<<grid, block, 0, stream>>>(s, rl, su, sv, k, n, first, count, out); break;
    case 1: reconstruct_kernel<K, 1><<<grid, block, 0, stream>>>(s, rl, su, sv, k, n, first, count, out); break;
    default: reconstruct_kernel<K, 2><<<grid, block, 0, stream>>>(s, rl, su, sv, k, n, first, count, out); break;
    }
    return hipGetLastError();
}

hipError_t launch_reconstruct(const void *src, int rl, const uint16_t *su, const uint16_t *sv, int bits, int cb,
                              size_t k, size_t n, size_t first, size_t count, uint16_t *out, hipStream_t stream) {
    switch (bits) {
    case 1: return launch_reconstruct_k<1>(src, rl, su, sv, cb, k, n, first, count, out, stream);
    case 2: return launch_reconstruct_k<2>(src, rl, su, sv, cb, k, n, first, count, out, stream);
    case 3: return launch_reconstruct_k<3>(src, rl, su, sv, cb, k, n, first, count, out, stream);
    case 4: return launch_reconstruct_k<4>(src, rl, su, sv, cb, k, n, first, count, out, stream);
    case 5: return launch_reconstruct_k<5>(src, rl, su, sv, cb, k, n, first, count, out, stream);
    case 6: return launch_reconstruct_k<6>(src, rl, su, sv, cb, k, n, first, count, out, stream);
    case 7: return launch_reconstruct_k<7>(src, rl, su, sv, cb, k, n, first, count, out, stream);
    default: return launch_reconstruct_k<8>(src, rl, su, sv, cb, k, n, first, count, out, stream);
    }
}

// ============================================================== get_rows
// GET_ROWS on records (src/exl3-ggml.cpp:19-49).  Workgroup (r, kb) writes
// out[r][128 kb .. +127] = column c = ids[r] % 128 of the original-basis
// reconstruct of record (ids[r] / 128, kb) as a 128x128 matrix, fp16-rounded
// (then widened for F32 output): decode into LDS (fp32), the H128 of each row
// over n restricted to the operations output c depends on (the same
// butterflies, in the same order, as the full transform: bit-exact), then the
// full H128 of that column over k and fp16((w * su) * sv) as exl3::reconstruct.
// An id outside [0, n) writes a NaN row and sets *bad_ids (if given) to 1.
template <int K, int CB>
__global__ __launch_bounds__(256) void get_rows_kernel(const uint8_t *__restrict__ records, size_t k, size_t n,
                                                       const int32_t *__restrict__ ids, void *__restrict__ out,
                                                       int out_f16, size_t out_stride, int *__restrict__ bad_ids) {
    constexpr int P = 129;
    __shared__ float blk[128 * P];
    __shared__ float colv[128];
    const int tid = threadIdx.x;
    const size_t r = blockIdx.x, kb = blockIdx.y;
    const int32_t id = ids[r];
    const size_t o = r * out_stride + kb * 128;
    if (id < 0 || (size_t)id >= n) {
        if (tid < 128) {
            if (out_f16) ((uint16_t *)out)[o + tid] = 0x7e00u;
            else ((uint32_t *)out)[o + tid] = 0x7fc00000u;
        }
        if (tid == 0 && kb == 0 && bad_ids) *bad_ids = 1;
        return;
    }
    const size_t nb = (size_t)id >> 7;
    const int c = id & 127;
#pragma unroll 1
    for (int i = 0; i < 4; ++i) {
        const int run = tid + 256 * i;
        const int tile = run >> 4, rc = run & 15;
        const int cr = rc & 7, h = rc >> 3, tr = tile >> 3, tc = tile & 7;
        const uint32_t *tp = tile_ptr<K>(records, 1, k, n, kb * 8 + tr, nb * 8 + tc);
        uint32_t w[RunGeo<K>::NW];
        load_run_words<K>(tp, cr, h, w);
        u4 a1, a2;
        decode_run<K, CB>(w, a1, a2);
        const uint32_t p1[4] = {a1.x, a1.y, a1.z, a1.w}, p2[4] = {a2.x, a2.y, a2.z, a2.w};
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int r0 = tr * 16 + run_slot_row(h, 2 * v), r1 = tr * 16 + run_slot_row(h, 2 * v + 1);
            const int cc = tc * 16 + cr;
            blk[r0 * P + cc] = half_bits_to_float((uint16_t)(p1[v] & 0xffffu));
            blk[r1 * P + cc] = half_bits_to_float((uint16_t)(p1[v] >> 16));
            blk[r0 * P + cc + 8] = half_bits_to_float((uint16_t)(p2[v] & 0xffffu));
            blk[r1 * P + cc + 8] = half_bits_to_float((uint16_t)(p2[v] >> 16));
        }
    }
    __syncthreads();
    // row tid: after the stage of stride 2^s only positions agreeing with c on
    // bits 0..s matter; v[m] holds position (m << (s + 1)) | (c & (2^(s+1) - 1))
    if (tid < 128) {
        const float *row = blk + tid * P;
        float v[64];
#pragma unroll
        for (int m = 0; m < 64; ++m) {
            const float a = row[2 * m], b = row[2 * m + 1];
            v[m] = (c & 1) ? a - b : a + b;
        }
#pragma unroll
        for (int s = 1; s < 7; ++s)
#pragma unroll
            for (int m = 0; m < (64 >> s); ++m) v[m] = ((c >> s) & 1) ? v[2 * m] - v[2 * m + 1] : v[2 * m] + v[2 * m + 1];
        colv[tid] = v[0] * 0.08838834764831844055f;
    }
    __syncthreads();
    if (tid < 64) {
        float e0 = colv[tid], e1 = colv[tid + 64];
        h128_wave(e0, e1, tid);
        const uint8_t *rec = records + (nb * (k >> 7) + kb) * group_bytes(K);
        const uint16_t *su = (const uint16_t *)(rec + 2048 * K);
        const float svc = half_bits_to_float(((const uint16_t *)(rec + 2048 * K + 256))[c]);
        const uint16_t h0 = float_to_half_bits(mul_rn_f32(mul_rn_f32(e0, half_bits_to_float(su[tid])), svc));
        const uint16_t h1 = float_to_half_bits(mul_rn_f32(mul_rn_f32(e1, half_bits_to_float(su[tid + 64])), svc));
        if (out_f16) {
            ((uint16_t *)out)[o + tid] = h0;
            ((uint16_t *)out)[o + tid + 64] = h1;
        } else {
            ((float *)out)[o + tid] = half_bits_to_float(h0);
            ((float *)out)[o + tid + 64] = half_bits_to_float(h1);
        }
    }
}

template <int K>
static hipError_t launch_get_rows_k(const void *records, int cb, size_t k, size_t n, const int32_t *ids, size_t count,
                                    void *out, int out_f16, size_t out_stride, int *bad_ids, hipStream_t stream) {
    const dim3 grid((unsigned)count, (unsigned)(k / 128)), block(256);
    const uint8_t *rec = (const uint8_t *)records;
    switch (cb) {
    case 0: get_rows_kernel<K, 0><<<grid, block, 0, stream>>>(rec, k, n, ids, out, out_f16, out_stride, bad_ids); break;
    case 1: get_rows_kernel<K, 1><<<grid, block, 0, stream>>>(rec, k, n, ids, out, out_f16, out_stride, bad_ids); break;
    default: get_rows_kernel<K, 2><<<grid, block, 0, stream>>>(rec, k, n, ids, out, out_f16, out_stride, bad_ids); break;
    }
    return hipGetLastError();
}

hipError_t launch_get_rows(const void *records, int bits, int cb, size_t k, size_t n, const int32_t *ids, size_t count,
                           void *out, int out_f16, size_t out_stride, int *bad_ids, hipStream_t stream) {
    switch (bits) {
    case 1: return launch_get_rows_k<1>(records, cb, k, n, ids, count, out, out_f16, out_stride, bad_ids, stream);
    case 2: return launch_get_rows_k<2>(records, cb, k, n, ids, count, out, out_f16, out_stride, bad_ids, stream);
    case 3: return launch_get_rows_k<3>(records, cb, k, n, ids, count, out, out_f16, out_stride, bad_ids, stream);
    case 4: return launch_get_rows_k<4>(records, cb, k, n, ids, count, out, out_f16, out_stride, bad_ids, stream);
    case 5: return launch_get_rows_k<5>(records, cb, k, n, ids, count, out, out_f16, out_stride, bad_ids, stream);
    case 6: return launch_get_rows_k<6>(records, cb, k, n, ids, count, out, out_f16, out_stride, bad_ids, stream);
    case 7: return launch_get_rows_k<7>(records, cb, k, n, ids, count, out, out_f16, out_stride, bad_ids, stream);
    default: return launch_get_rows_k<8>(records, cb, k, n, ids, count, out, out_f16, out_stride, bad_ids, stream);
    }
}

// ============================================================== records
// One workgroup per record (nb, kb): 64 tiles (tile (r, c) <- upstream tile
// (8 kb + r, 8 nb + c)), then su[128 kb ..], sv[128 nb ..].
__global__ __launch_bounds__(256) void pack_records_kernel(const uint16_t *__restrict__ packed,
                                                           const uint16_t *__restrict__ su,
                                                           const uint16_t *__restrict__ sv, int bits, size_t k,
                                                           size_t n, uint8_t *__restrict__ records) {
    const size_t kbs = k / 128, rec_id = blockIdx.x;
    const size_t nb = rec_id / kbs, kb = rec_id - nb * kbs;
    uint8_t *g = records + rec_id * group_bytes(bits);
    const int tile_u4 = 2 * bits;  // 32*bits bytes per tile = 2*bits uint4
    for (int i = threadIdx.x; i < 64 * tile_u4; i += blockDim.x) {
        const int t = i / tile_u4, o = i - t * tile_u4;
        const size_t up = (kb * 8 + (t >> 3)) * (n / 16) + nb * 8 + (t & 7);
        ((uint4 *)g)[i] = ((const uint4 *)(packed + up * 16 * bits))[o];
    }
    if (threadIdx.x < 16) ((uint4 *)(g + 2048 * bits))[threadIdx.x] = ((const uint4 *)(su + kb * 128))[threadIdx.x];
    else if (threadIdx.x < 32)
        ((uint4 *)(g + 2048 * bits + 256))[threadIdx.x - 16] = ((const uint4 *)(sv + nb * 128))[threadIdx.x - 16];
}

hipError_t launch_pack_records(const uint16_t *packed, const uint16_t *su, const uint16_t *sv, int bits, size_t k,
                               size_t n, void *records, hipStream_t stream) {
    const size_t recs = (k / 128) * (n / 128);
    pack_records_kernel<<<dim3((unsigned)recs), dim3(256), 0, stream>>>(packed, su, sv, bits, k, n,
                                                                         (uint8_t *)records);
    return hipGetLastError();
}

__global__ void set_one_kernel(int *p) { *p = 1; }

// patches/llama-exl3.patch:327-338: a scale is invalid when its exponent field is all ones
__global__ __launch_bounds__(256) void validate_kernel(const uint8_t *__restrict__ records, int bits,
                                                       int *__restrict__ result) {
    const uint16_t *s = (const uint16_t *)(records + (size_t)blockIdx.x * group_bytes(bits) + 2048 * bits);
    if ((s[threadIdx.x] & 0x7c00u) == 0x7c00u) *result = 0;
}

hipError_t launch_validate(const void *records, size_t nrecords, int bits, int *result, hipStream_t stream) {
    set_one_kernel<<<1, 1, 0, stream>>>(result);
    if (nrecords) validate_kernel<<<dim3((unsigned)nrecords), dim3(256), 0, stream>>>((const uint8_t *)records, bits, result);
    return hipGetLastError();
}

// ============================================================== activations
__device__ __forceinline__ float load_x(const void *x, int x_f16, size_t stride, size_t r, size_t i) {
    if (x_f16) return half_bits_to_float(((const uint16_t *)x)[r * stride + i]);
    return ((const float *)x)[r * stride + i];
}

// ============================================================== GEMV
// One launch per call.  Workgroup (nb, split s) owns the 128-row blocks
// kb in [kb0, kb1) of the 128-column group nb.  A group is tile rows
// 4 r4 .. 4 r4 + 3 x tile columns 2 c2, 2 c2 + 1 of record (nb, kb); wave w
// owns column pair c2 = w % 4 and, with P = waves / 4, the groups
// (kb, r4) numbered q = 2 (kb - kb0) + r4 with q % P = w / 4.
//   1. prep: xh[r] = H128(x[r] * su) in fp32 (su from record (0, kb),
//      src/exl3-ggml.cpp:60-73) for every (kb, r) of the workgroup, split into
//      fp16 hi = rn(xh) and lo = rn(xh - hi) and stored in LDS as MFMA B
//      fragments: column m < 8 carries hi of row m, column m >= 8 lo of row m - 8.
//      All activation loads of a wave are in flight together.
//   2. weight stream: lane l = 16 g + i loads chunk i % 8 (K contiguous words)
//      of tile (4 r4 + g, 2 c2 + i / 8): one K-word load per lane and group,
//      DEPTH groups in flight, all issued after the prep barrier: weight loads
//      issued earlier delay the activation loads of the other workgroups behind
//      them (measured: 3 groups before the barrier cost 4 % at k = 14336, all 8
//      cost 11 %), and the prep is on every workgroup's critical path.
//   3. a lane decodes its chunk's 32 weights in registers (the first states
//      reach into the previous chunk's last word, taken from the neighbouring
//      lane with DPP) into four MFMA A fragments (rows 0-7 / 8-15 of its tile row
//      for columns j and j + 8 of its tile, j = i % 8); four 16x16x32 MFMAs per
//      group accumulate D1 (A row i -> column 32 c2 + i for i < 8, 32 c2 + 8 + i
//      otherwise) and D2 (32 c2 + 8 + i; 32 c2 + 16 + i).  D[n][m]: lane l holds
//      m = l % 16, n = 4 (l / 16) + e.
//   4. epilogue: hi + lo, the P partials of each column pair summed in LDS;
//      split-K partials are reduced in split order by the last workgroup of
//      the column group, which applies H128 and sv (src/exl3-ggml.cpp:84-90).
template <int K>
struct GemvStream {
    static constexpr int DEPTH = K <= 2 ? 12 : (K <= 4 ? 8 : 4);  // groups in flight per wave
};
constexpr int kGemvPrepMax = 16;          // a workgroup preps at most kGemvPrepMax x waves (kb, row) blocks
constexpr size_t kGemvDummyBytes = 8192;  // >= largest lane offset of a group + its K words (1024 K)
constexpr size_t kGemvFragLds = 49152;    // LDS budget of the B fragments of a workgroup (rows <= 8)
constexpr size_t kGemvFragLds16 = 65536;  // the same for rows 9..16 (two workgroups still fit a CU)

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

// MODE 0 (rows 1..8): one block of 16 B columns, hi and lo of 8 rows.
// MODE 1 (rows 9..16): a second block of B columns carries rows 8..15 (hi and lo as
// for rows 0..7); each decoded A fragment feeds both blocks' MFMAs, so the decode
// is shared by all 16 rows.
// MODE 2 (rows 17..32): two blocks of 16 rows each, fp16 activations without the
// lo halves, prepared once per call by gemv_xprep_kernel (xpre) and copied into
// LDS instead of being transformed again by every column group.
template <int K, int CB, int MODE>
__global__ __launch_bounds__(kGemvWaves * 64) void gemv_kernel(
    GemvTargets tg, int kbs, int splits, int kq, int kr, const void *__restrict__ x, int x_f16, size_t x_stride,
    int rows, const uint8_t *__restrict__ dummy, float *__restrict__ partials, unsigned *__restrict__ counters,
    int y_f16, const uint8_t *__restrict__ xpre) {
    constexpr bool TWO = MODE >= 1, HILO = MODE <= 1;
    constexpr int W = kGemvWaves;
    constexpr int P = W / 4;  // waves per column pair
    constexpr int NT = W * 64;
    constexpr size_t GB = (size_t)2048 * K + 512;
    // rows 9..16 need 8 more accumulator and fragment registers: a shorter ring at
    // K <= 2 keeps them within 128 VGPRs (two workgroups per CU)
    constexpr int D = TWO && K <= 2 ? 8 : GemvStream<K>::DEPTH;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ int last_flag;
    uint8_t *frag = smem;
    // B fragments of one (kb, r4, half): [kg][hl][row] x 16 bytes (MODE 2: [kg][row])
    const int blk_bytes = (HILO ? 128 : 64) * rows;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int cp = wave & 3, part = wave >> 2;
    // grid (column group, split): no division on the way to the first loads.
    // Split s owns kq + (s < kr) records from kb0 (kq = kbs / splits, kr = kbs % splits)
    const int nb = blockIdx.x, s = blockIdx.y;
    const int kb0 = s * kq + (s < kr ? s : kr), kb1 = kb0 + kq + (s < kr ? 1 : 0);
    const int nkb = kb1 - kb0;
    // the matrix of column group nb (targets share k, x and the bit rate)
    int mi = 0;
#pragma unroll
    for (int i = 1; i < kGemvMaxTargets; ++i)
        if (i < tg.count && nb >= tg.nb_end[i - 1]) mi = i;
    const uint8_t *records = tg.records[0];
    void *y = tg.y[0];
    size_t y_stride = tg.y_stride[0];
    const void *res = tg.res[0];
    size_t res_stride = tg.res_stride[0];
    int nbl = nb;  // column group within the matrix
#pragma unroll
    for (int i = 1; i < kGemvMaxTargets; ++i)
        if (mi == i) {
            records = tg.records[i];
            y = tg.y[i];
            y_stride = tg.y_stride[i];
            res = tg.res[i];
            res_stride = tg.res_stride[i];
            nbl = nb - tg.nb_end[i - 1];
        }
    const uint8_t *colgroup = records + (size_t)nbl * kbs * GB;

    // output scales for the epilogue (record (nb, 0), src/exl3-ggml.cpp:84-85)
    const uint16_t *svp = (const uint16_t *)(colgroup + 2048 * K + 256);

    // weight stream: this wave's groups are q = part + P i; issues past its
    // last group read the workspace's dummy region, so every issue is
    // unconditional and the compiler's wait counts stay exact
    const int g = lane >> 4, li = lane & 15, j = li & 7;
    const uint32_t lane_off = (uint32_t)(((8 * g + 2 * cp + (li >> 3)) * 32 + 4 * j) * K);
    const int ngroups = (2 * nkb - part + P - 1) / P;
    auto group_q = [&](int i) { return part + P * i; };
    auto group_src = [&](int i) -> const uint8_t * {
        const int q = group_q(i);
        return i < ngroups ? colgroup + (size_t)(kb0 + (q >> 1)) * GB + (size_t)(q & 1) * 1024 * K + lane_off
                           : dummy + lane_off;
    };
    uint32_t buf[D][K];

    // 1-2. prep: xh = H128(x[r] su) per (kb, row) block of the workgroup, as
    // fp16 hi = rn(xh) and lo = rn(xh - hi) into the B fragments.  Unit q of
    // wave w is up to four blocks (block = kbl rows + r): lane 16 g + l holds
    // elements 8 i .. 8 i + 7, i = h128_lane_block(l), of block (4 q + g) W + w
    // (blocks dealt across the waves first, so a few blocks still run on as many
    // waves): H128 stages 1, 2, 4 inside the lane, 8 .. 64 with the lanes holding
    // i ^ 1, 2, 4, 8 (one DPP read each), in the reference's stage order.
    // Elements 8 i .. 8 i + 7 are one 16-byte slot of the fragment blocks (tile
    // row 4 (i / 8) + (i / 2) % 4 ... : r4 = i / 8, kg = (i / 2) % 4, half = i % 2),
    // so a lane stores hi and lo with one 16-byte write each.  NQ (units per
    // wave) is a compile-time bound, and a block past the last re-reads the last
    // block (never stored), so the loads are straight-line code and all in
    // flight together.
    const int nblk = nkb * rows;
    auto prologue = [&](auto nq_c, auto is_f16) {
        constexpr int NQ = decltype(nq_c)::value;
        constexpr bool XF16 = decltype(is_f16)::value;
        const int pi = h128_lane_block(lane & 15);  // this lane's 8-element block of each unit
        uint4 xr[NQ][XF16 ? 1 : 2], sr[NQ];
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int bu = (4 * q + g) * W + wave;
            const int blk = bu < nblk ? bu : nblk - 1;
            const int kbl = blk / rows, r = blk - kbl * rows;
            const int kb = kb0 + kbl;
            sr[q] = *(const uint4 *)(records + (size_t)kb * GB + 2048 * K + 16 * pi);  // record (0, kb): su
            const size_t xi = (size_t)r * x_stride + (size_t)kb * 128 + 8 * pi;
            // element alignment only (any row stride): the compiler emits unaligned vector loads
            if constexpr (XF16) __builtin_memcpy(&xr[q][0], (const uint16_t *)x + xi, 16);
            else __builtin_memcpy(&xr[q][0], (const float *)x + xi, 32);
        }
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            if (4 * q * W + wave < nblk) {  // uniform in the wave: the DPP stages see every lane
                const uint32_t sw[4] = {sr[q].x, sr[q].y, sr[q].z, sr[q].w};
                float v[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    float xv;
                    if constexpr (XF16) {
                        const uint4 &w4 = xr[q][0];
                        const uint32_t wd = (j >> 1) == 0 ? w4.x : (j >> 1) == 1 ? w4.y : (j >> 1) == 2 ? w4.z : w4.w;
                        xv = half_bits_to_float((uint16_t)(wd >> (16 * (j & 1))));
                    } else {
                        const uint4 &w4 = xr[q][j >> 2];
                        const uint32_t wd = (j & 3) == 0 ? w4.x : (j & 3) == 1 ? w4.y : (j & 3) == 2 ? w4.z : w4.w;
                        xv = __uint_as_float(wd);
                    }
                    v[j] = xv * half_bits_to_float((uint16_t)(sw[j >> 1] >> (16 * (j & 1))));
                }
#pragma unroll
                for (int st = 1; st < 8; st <<= 1)
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        if (!(j & st)) {
                            const float a = v[j], b = v[j | st];
                            v[j] = a + b;
                            v[j | st] = a - b;
                        }
                auto lane_stage = [&](auto sc) {
                    constexpr int S = decltype(sc)::value;
                    const float sgn = (pi & S) ? -1.f : 1.f;
                    float pv[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) pv[j] = dpp_block_xor<S>(v[j]);
#pragma unroll
                    for (int j = 0; j < 8; ++j) v[j] = __builtin_fmaf(v[j], sgn, pv[j]);
                };
                lane_stage(std::integral_constant<int, 1>{});
                lane_stage(std::integral_constant<int, 2>{});
                lane_stage(std::integral_constant<int, 4>{});
                lane_stage(std::integral_constant<int, 8>{});
                const int blk = (4 * q + g) * W + wave;
                if (blk < nblk) {
                    const int kbl = blk / rows, r = blk - kbl * rows;
                    h8 hi, lo;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const float e = v[j] * 0.08838834764831844055f;
                        hi[j] = (_Float16)e;
                        lo[j] = (_Float16)(e - (float)hi[j]);
                    }
                    const int r4 = pi >> 3, kg = (pi >> 1) & 3, half = pi & 1;
                    uint8_t *bp = frag + (size_t)((kbl * 2 + r4) * 2 + half) * blk_bytes;
                    *(h8 *)(bp + ((kg * 2 + 0) * rows + r) * 16) = hi;
                    *(h8 *)(bp + ((kg * 2 + 1) * rows + r) * 16) = lo;
                }
            }
        }
    };
    // at most one block per wave (rows 1 and short k): one block per wave with
    // 2 elements per lane (stride 1 inside the lane, 2 .. 64 across all 64
    // lanes) is faster than putting the blocks on 16-lane rows of fewer waves
    auto prologue_one = [&](auto is_f16) {
        constexpr bool XF16 = decltype(is_f16)::value;
        const int blk = wave < nblk ? wave : nblk - 1;
        const int kbl = blk / rows, r = blk - kbl * rows;
        const int kb = kb0 + kbl;
        const uint32_t ps = ((const uint32_t *)(records + (size_t)kb * GB + 2048 * K))[lane];  // su pair
        const size_t xi = (size_t)r * x_stride + (size_t)kb * 128 + 2 * lane;
        float a, b;
        if constexpr (XF16) {
            a = half_bits_to_float(((const uint16_t *)x)[xi]);
            b = half_bits_to_float(((const uint16_t *)x)[xi + 1]);
        } else {
            a = ((const float *)x)[xi];
            b = ((const float *)x)[xi + 1];
        }
        if (wave < nblk) {
            a *= half_bits_to_float((uint16_t)(ps & 0xffffu));
            b *= half_bits_to_float((uint16_t)(ps >> 16));
            h128_pair(a, b, lane);
            // elements 2 lane (+1): r4 = lane / 32, kg = lane / 8 % 4, half = lane / 4 % 2,
            // position 2 (lane % 4) (+1) of the 16-byte slot
            const _Float16 ha = (_Float16)a, hb = (_Float16)b;
            const h2 hi = {ha, hb}, lo = {(_Float16)(a - (float)ha), (_Float16)(b - (float)hb)};
            const int r4 = lane >> 5, kg = (lane >> 3) & 3, half = (lane >> 2) & 1, jj = 2 * (lane & 3);
            uint8_t *bp = frag + (size_t)((kbl * 2 + r4) * 2 + half) * blk_bytes + jj * 2;
            *(h2 *)(bp + ((kg * 2 + 0) * rows + r) * 16) = hi;
            *(h2 *)(bp + ((kg * 2 + 1) * rows + r) * 16) = lo;
        }
    };
    auto prologue_x = [&](auto is_f16) {
        const int nq = (nblk + 4 * W - 1) / (4 * W);  // units of wave 0 (the most)
        if (nblk <= W) prologue_one(is_f16);
        else if (nq <= 1) prologue(std::integral_constant<int, 1>{}, is_f16);
        else if (nq <= 2) prologue(std::integral_constant<int, 2>{}, is_f16);
        else prologue(std::integral_constant<int, 4>{}, is_f16);
    };
    if constexpr (MODE == 2) {
        // the workgroup's records [kb0, kb1) of the target's prepared activations,
        // laid out exactly as the LDS fragments: one contiguous copy, all loads first
        const uint8_t *src = xpre + ((size_t)mi * kbs + kb0) * (size_t)(4 * blk_bytes);
        const int nbytes = nkb * 4 * blk_bytes;  // <= kGemvFragLds16
        constexpr int CPY = (int)(kGemvFragLds16 / (NT * 16));
        u4 cv[CPY];
#pragma unroll
        for (int c = 0; c < CPY; ++c) {
            const int o = (c * NT + tid) * 16;
            if (o < nbytes) cv[c] = *(const u4 *)(src + o);
        }
#pragma unroll
        for (int c = 0; c < CPY; ++c) {
            const int o = (c * NT + tid) * 16;
            if (o < nbytes) *(u4 *)(frag + o) = cv[c];
        }
    } else {
        if (x_f16) prologue_x(std::true_type{});
        else prologue_x(std::false_type{});
    }
    const float sv0 = half_bits_to_float(svp[lane]), sv1 = half_bits_to_float(svp[lane + 64]);
    __syncthreads();
#pragma unroll
    for (int d = 0; d < D; ++d) load_chunk<K>(group_src(d), buf[d]);

    // 4. decode + MFMA.  B operand lane l: m = l % 16 -> (hl, row) = (m / 8, m % 8),
    // k group l / 16; rows >= `rows` read the last row (their columns are discarded)
    // (MODE 2: m -> row m, and row 16 + m in the second block)
    const int m = li, hl = m >> 3;
    const int r1 = HILO ? (m & 7) : m, r2 = HILO ? 8 + (m & 7) : 16 + m;
    const int mrow = r1 < rows ? r1 : rows - 1, mrow2 = r2 < rows ? r2 : rows - 1;  // TWO: the second block
    const int boff = (HILO ? (g * 2 + hl) * rows + mrow : g * rows + mrow) * 16;
    const int boff2 = (HILO ? (g * 2 + hl) * rows + mrow2 : g * rows + mrow2) * 16;
    const bool first_chunk = j == 0;
    f4 acc1 = {0.f, 0.f, 0.f, 0.f}, acc2 = {0.f, 0.f, 0.f, 0.f};
    f4 acc3 = {0.f, 0.f, 0.f, 0.f}, acc4 = {0.f, 0.f, 0.f, 0.f};  // TWO: acc1 / acc2 of rows 8..15
    auto mac = [&](int i, const uint32_t (&w)[K]) {
        // last word of the previous chunk of the same tile: lane i - 1, or i + 7 for chunk 0
        const uint32_t p1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)w[K - 1], 0x121, 0xF, 0xF, false);  // row_ror:1
        const uint32_t p9 = (uint32_t)__builtin_amdgcn_mov_dpp((int)w[K - 1], 0x129, 0xF, 0xF, false);  // row_ror:9
        u4 fr[4];
        decode_chunk<K, CB>(w, first_chunk ? p9 : p1, fr);
        const uint8_t *bp = frag + (size_t)group_q(i) * 2 * blk_bytes + boff;
        const h8 blo = *(const h8 *)bp, bhi = *(const h8 *)(bp + blk_bytes);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(bitcast<h8>(fr[0]), blo, acc1, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(bitcast<h8>(fr[1]), bhi, acc1, 0, 0, 0);
        acc2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(bitcast<h8>(fr[2]), blo, acc2, 0, 0, 0);
        acc2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(bitcast<h8>(fr[3]), bhi, acc2, 0, 0, 0);
        if constexpr (TWO) {
            const uint8_t *bp2 = frag + (size_t)group_q(i) * 2 * blk_bytes + boff2;
            const h8 clo = *(const h8 *)bp2, chi = *(const h8 *)(bp2 + blk_bytes);
            acc3 = __builtin_amdgcn_mfma_f32_16x16x32_f16(bitcast<h8>(fr[0]), clo, acc3, 0, 0, 0);
            acc3 = __builtin_amdgcn_mfma_f32_16x16x32_f16(bitcast<h8>(fr[1]), chi, acc3, 0, 0, 0);
            acc4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(bitcast<h8>(fr[2]), clo, acc4, 0, 0, 0);
            acc4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(bitcast<h8>(fr[3]), chi, acc4, 0, 0, 0);
        }
    };
    int i0 = 0;
    for (; i0 + D <= ngroups; i0 += D) {  // full rounds: no branches between issue and use
#pragma unroll
        for (int d = 0; d < D; ++d) {
            mac(i0 + d, buf[d]);
            // refill a slot once its words are decoded: loading into registers
            // still being read would make the compiler rotate the ring with
            // copies, and a copy of an in-flight load waits for it
            load_chunk<K>(group_src(i0 + d + D), buf[d]);
        }
    }
#pragma unroll
    for (int d = 0; d < D; ++d)  // tail: fewer than D groups, already in flight
        if (i0 + d < ngroups) mac(i0 + d, buf[d]);

    // 5. epilogue: hi + lo (MFMA column m < 8 gets column m + 8) into this wave's
    // 32 columns of its share of the workgroup partial (MODE 2: column m is row m)
    __syncthreads();  // every wave is done with the fragments; LDS now holds the partials
    float *red = (float *)smem;  // [P][rows][128]
    const int nval = rows * 128;
#pragma unroll
    for (int e = 0; e < 4 && !HILO; ++e) {
        const int n = 4 * g + e;
        if (m < rows) {
            float *rp = red + part * nval + m * 128 + 32 * cp;
            rp[n < 8 ? n : 8 + n] = acc1[e];
            rp[n < 8 ? 8 + n : 16 + n] = acc2[e];
        }
        if (16 + m < rows) {
            float *rp = red + part * nval + (16 + m) * 128 + 32 * cp;
            rp[n < 8 ? n : 8 + n] = acc3[e];
            rp[n < 8 ? 8 + n : 16 + n] = acc4[e];
        }
    }
#pragma unroll
    for (int e = 0; e < 4 && HILO; ++e) {
        const int n = 4 * g + e;
        const float o1 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc1[e]), 0x108, 0xF, 0xF, true));
        const float o2 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc2[e]), 0x108, 0xF, 0xF, true));
        if (m < 8 && m < rows) {
            float *rp = red + part * nval + m * 128 + 32 * cp;
            rp[n < 8 ? n : 8 + n] = acc1[e] + o1;
            rp[n < 8 ? 8 + n : 16 + n] = acc2[e] + o2;
        }
        if constexpr (TWO) {
            const float o3 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc3[e]), 0x108, 0xF, 0xF, true));
            const float o4 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc4[e]), 0x108, 0xF, 0xF, true));
            if (m < 8 && 8 + m < rows) {
                float *rp = red + part * nval + (8 + m) * 128 + 32 * cp;
                rp[n < 8 ? n : 8 + n] = acc3[e] + o3;
                rp[n < 8 ? 8 + n : 16 + n] = acc4[e] + o4;
            }
        }
    }
    __syncthreads();
    constexpr int PER = ((MODE == 2 ? 32 : MODE == 1 ? 16 : 8) * 128 + NT - 1) / NT;
    float psum[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int t = tid + i * NT;
        float v = 0.f;
        if (t < nval) {
#pragma unroll
            for (int pp = 0; pp < P; ++pp) v += red[pp * nval + t];
        }
        psum[i] = v;
    }
    // output of row rr from its sums a0 (element lane) and a1 (lane + 64): H128
    // over the 128 columns, sv (src/exl3-ggml.cpp:84-90), the optional residual
    auto finish_row = [&](int rr, float a0, float a1) {
        h128_wave(a0, a1, lane);
        a0 *= sv0;
        a1 *= sv1;
        const size_t o = (size_t)rr * y_stride + (size_t)nbl * 128;
        if (res) {  // fused residual: y = res + layer, one rounding
            const size_t ro = (size_t)rr * res_stride + (size_t)nbl * 128;
            if (y_f16) {
                a0 += half_bits_to_float(((const uint16_t *)res)[ro + lane]);
                a1 += half_bits_to_float(((const uint16_t *)res)[ro + lane + 64]);
            } else {
                a0 += ((const float *)res)[ro + lane];
                a1 += ((const float *)res)[ro + lane + 64];
            }
        }
        if (y_f16) {
            ((uint16_t *)y)[o + lane] = float_to_half_bits(a0);
            ((uint16_t *)y)[o + lane + 64] = float_to_half_bits(a1);
        } else {
            ((float *)y)[o + lane] = a0;
            ((float *)y)[o + lane + 64] = a1;
        }
    };
    if (splits > 1) {
        float *mine = partials + ((size_t)nb * splits + s) * (size_t)nval;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int t = tid + i * NT;
            if (t < nval) store_coherent(mine + t, psum[i]);
        }
        if (!arrive_last(counters + nb, (unsigned)splits, &last_flag)) return;
        // the last workgroup: wave r sums row r's elements lane and lane + 64 over
        // the splits in split order (so the result does not depend on which
        // workgroup arrived last), all of a lane's loads in flight together,
        // straight into the registers of the output transform
        const float *all = partials + (size_t)nb * splits * (size_t)nval;
        for (int rr = wave; rr < rows; rr += W) {
            constexpr int B = 16;
            float a0 = 0.f, a1 = 0.f;
            for (int base = 0; base < splits; base += B) {
                float v0[B], v1[B];
#pragma unroll
                for (int jb = 0; jb < B; ++jb) {
                    const int sp = base + jb < splits ? base + jb : splits - 1;  // repeats are not added
                    const float *q = all + (size_t)sp * nval + rr * 128 + lane;
                    v0[jb] = load_coherent(q);
                    v1[jb] = load_coherent(q + 64);
                }
#pragma unroll
                for (int jb = 0; jb < B; ++jb)
                    if (base + jb < splits) {
                        a0 += v0[jb];
                        a1 += v1[jb];
                    }
            }
            finish_row(rr, a0, a1);
        }
        if (tid == 0) reset_counter(counters + nb);  // self-reset for the next call
        return;
    }
    // 6. (one workgroup per column group) output H128 per row from the LDS sums
    float *ybuf = red + P * nval;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int t = tid + i * NT;
        if (t < nval) ybuf[t] = psum[i];
    }
    __syncthreads();
    for (int rr = wave; rr < rows; rr += W) finish_row(rr, ybuf[rr * 128 + lane], ybuf[rr * 128 + lane + 64]);
}

// Activations of the 17..32-row GEMV (MODE 2): fp16(H128(x[r] su)), su from record
// (0, kb) of target t (src/exl3-ggml.cpp:60-73), in gemv_kernel's LDS fragment
// order without lo halves: [t][kb][r4][half][kg][row] x 16 bytes.  One wave per
// (row, kb, target); lane l holds elements 2 l and 2 l + 1 (h128_pair).
__global__ __launch_bounds__(256) void gemv_xprep_kernel(GemvTargets tg, int bits, const void *__restrict__ x,
                                                         int x_f16, size_t x_stride, int rows, int kbs,
                                                         uint16_t *__restrict__ xpre) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6), kb = blockIdx.y, t = blockIdx.z;
    if (r >= rows) return;  // whole waves
    const uint8_t *records = tg.records[0];
#pragma unroll
    for (int i = 1; i < kGemvMaxTargets; ++i)
        if (t == i) records = tg.records[i];
    const uint32_t ps = ((const uint32_t *)(records + (size_t)kb * group_bytes(bits) + 2048 * bits))[lane];
    const size_t xi = (size_t)r * x_stride + (size_t)kb * 128 + 2 * lane;
    float a, b;
    if (x_f16) {
        a = half_bits_to_float(((const uint16_t *)x)[xi]);
        b = half_bits_to_float(((const uint16_t *)x)[xi + 1]);
    } else {
        a = ((const float *)x)[xi];
        b = ((const float *)x)[xi + 1];
    }
    a *= half_bits_to_float((uint16_t)(ps & 0xffffu));
    b *= half_bits_to_float((uint16_t)(ps >> 16));
    h128_pair(a, b, lane);
    // elements 2 lane (+1): r4 = lane / 32, kg = lane / 8 % 4, half = lane / 4 % 2,
    // position 2 (lane % 4) (+1) of the 16-byte slot
    const int r4 = lane >> 5, kg = (lane >> 3) & 3, half = (lane >> 2) & 1;
    uint16_t *dst = xpre + ((((size_t)t * kbs + kb) * 2 + r4) * 2 + half) * (size_t)(32 * rows) + (kg * rows + r) * 8 +
                    2 * (lane & 3);
    *(uint32_t *)dst = (uint32_t)float_to_half_bits(a) | ((uint32_t)float_to_half_bits(b) << 16);
}

// B-fragment bytes of one record in a GEMV workgroup's LDS (hi and lo halves up to
// 16 rows, fp16 only above)
static size_t gemv_frag_bytes_per_kb(size_t rows) { return (rows > 16 ? 256 : 512) * rows; }

// LDS bytes of a GEMV workgroup: its B fragments, reused after the main loop for
// the P partials and the output rows
static size_t gemv_lds_bytes(int nkb_max, size_t rows) {
    const size_t frag = (size_t)nkb_max * gemv_frag_bytes_per_kb(rows);
    const size_t red = (size_t)(kGemvWaves / 4 + 1) * rows * 128 * 4;
    return ((frag > red ? frag : red) + 15) & ~(size_t)15;
}

GemvPlan gemv_plan(size_t k, size_t n, size_t rows) {
    GemvPlan p{};
    p.nbs = (int)(n / 128);
    p.kbs = (int)(k / 128);
    // about four records per workgroup (a workgroup's fixed latency chain then
    // stays small against its stream), between 128 and 512 workgroups (one to two
    // per CU); measured best or within 10 % of best for k = 2048..14336
    int s = (p.kbs + 3) / 4;
    if (p.nbs * s > 512) s = 512 / p.nbs;
    if (p.nbs * s < 128) s = (128 + p.nbs - 1) / p.nbs;
    s = s < 1 ? 1 : (s > p.kbs ? p.kbs : s);
    // a workgroup's B fragments must fit its LDS budget and a wave prepares at
    // most kGemvPrepMax (kb, row) blocks; one kb per workgroup always fits
    for (;;) {
        const size_t nkb = ((size_t)p.kbs + s - 1) / s;
        const bool ok_lds = nkb * gemv_frag_bytes_per_kb(rows) <= (rows > 8 ? kGemvFragLds16 : kGemvFragLds);
        // above 16 rows the activations are prepared once per call (gemv_xprep_kernel)
        const bool ok_prep = rows > 16 || (nkb * rows + kGemvWaves - 1) / kGemvWaves <= (size_t)kGemvPrepMax;
        if ((ok_lds && ok_prep) || s >= p.kbs) break;
        ++s;
    }
    p.splits = s;
    p.nkw = (p.kbs + s - 1) / s;
    size_t off = 0;
    p.counters_off = off;
    off += counter_region_bytes(n);
    p.dummy_off = off;  // target of the stream's issues past a wave's last group (loaded, never used)
    off += kGemvDummyBytes;
    p.partials_off = off;
    if (s > 1) off += (size_t)p.nbs * s * rows * 128 * 4;
    off = (off + 255) & ~(size_t)255;
    p.xpre_off = off;  // rows > 16: prepared activations of up to kGemvMaxTargets matrices
    if (rows > 16) off += (size_t)kGemvMaxTargets * p.kbs * gemv_frag_bytes_per_kb(rows);
    p.bytes = (off + 255) & ~(size_t)255;
    return p;
}

template <int K, int CB>
static hipError_t launch_gemv_kc(const GemvTargets &tg, const void *x, int x_f16, size_t rows, size_t x_stride,
                                 int y_f16, uint8_t *ws, const GemvPlan &p, hipStream_t stream) {
    const size_t lds = gemv_lds_bytes(p.nkw, rows);
    // x fastest: workgroup (nb, s) is dispatched as nb + s nbs, as a 1-D grid would be
    const dim3 grid((unsigned)p.nbs, (unsigned)p.splits), block(kGemvWaves * 64);
    const int kq = p.kbs / p.splits, kr = p.kbs % p.splits;
    float *part = (float *)(ws + p.partials_off);
    unsigned *cnt = (unsigned *)(ws + p.counters_off);
    if (rows > 16) {
        uint16_t *xp = (uint16_t *)(ws + p.xpre_off);
        gemv_xprep_kernel<<<dim3((unsigned)((rows + 3) / 4), (unsigned)p.kbs, (unsigned)tg.count), dim3(256), 0,
                            stream>>>(tg, K, x, x_f16, x_stride, (int)rows, p.kbs, xp);
        gemv_kernel<K, CB, 2><<<grid, block, lds, stream>>>(tg, p.kbs, p.splits, kq, kr, x, x_f16, x_stride,
                                                            (int)rows, ws + p.dummy_off, part, cnt, y_f16,
                                                            (const uint8_t *)xp);
    } else if (rows > 8) {
        gemv_kernel<K, CB, 1><<<grid, block, lds, stream>>>(tg, p.kbs, p.splits, kq, kr, x, x_f16, x_stride,
                                                            (int)rows, ws + p.dummy_off, part, cnt, y_f16, nullptr);
    } else {
        gemv_kernel<K, CB, 0><<<grid, block, lds, stream>>>(tg, p.kbs, p.splits, kq, kr, x, x_f16, x_stride,
                                                            (int)rows, ws + p.dummy_off, part, cnt, y_f16, nullptr);
    }
    return hipGetLastError();
}

template <int K>
static hipError_t launch_gemv_k(const GemvTargets &tg, int cb, const void *x, int x_f16, size_t rows, size_t x_stride,
                                int y_f16, uint8_t *ws, const GemvPlan &p, hipStream_t stream) {
    switch (cb) {
    case 0: return launch_gemv_kc<K, 0>(tg, x, x_f16, rows, x_stride, y_f16, ws, p, stream);
    case 1: return launch_gemv_kc<K, 1>(tg, x, x_f16, rows, x_stride, y_f16, ws, p, stream);
    default: return launch_gemv_kc<K, 2>(tg, x, x_f16, rows, x_stride, y_f16, ws, p, stream);
    }
}

hipError_t launch_gemv_targets(const GemvTargets &tg, int bits, int cb, const void *x, int x_f16, size_t rows,
                               size_t x_stride, int y_f16, void *workspace, const GemvPlan &p, hipStream_t stream) {
    uint8_t *ws = (uint8_t *)workspace;
    switch (bits) {
    case 1: return launch_gemv_k<1>(tg, cb, x, x_f16, rows, x_stride, y_f16, ws, p, stream);
    case 2: return launch_gemv_k<2>(tg, cb, x, x_f16, rows, x_stride, y_f16, ws, p, stream);
    case 3: return launch_gemv_k<3>(tg, cb, x, x_f16, rows, x_stride, y_f16, ws, p, stream);
    case 4: return launch_gemv_k<4>(tg, cb, x, x_f16, rows, x_stride, y_f16, ws, p, stream);
    case 5: return launch_gemv_k<5>(tg, cb, x, x_f16, rows, x_stride, y_f16, ws, p, stream);
    case 6: return launch_gemv_k<6>(tg, cb, x, x_f16, rows, x_stride, y_f16, ws, p, stream);
    case 7: return launch_gemv_k<7>(tg, cb, x, x_f16, rows, x_stride, y_f16, ws, p, stream);
    default: return launch_gemv_k<8>(tg, cb, x, x_f16, rows, x_stride, y_f16, ws, p, stream);
    }
}

hipError_t launch_gemv(const void *records, int bits, int cb, size_t k, size_t n, const void *x, int x_f16,
                       size_t rows, size_t x_stride, void *y, int y_f16, size_t y_stride, void *workspace,
                       const GemvPlan &p, hipStream_t stream, const void *res, size_t res_stride) {
    (void)k;
    GemvTargets tg{};
    tg.records[0] = (const uint8_t *)records;
    tg.y[0] = y;
    tg.y_stride[0] = y_stride;
    tg.res[0] = res;
    tg.res_stride[0] = res_stride;
    tg.nb_end[0] = (int)(n / 128);
    tg.count = 1;
    return launch_gemv_targets(tg, bits, cb, x, x_f16, rows, x_stride, y_f16, workspace, p, stream);
}

// ============================================================== GEMM
// Activation prep for the GEMM: xh = fp16(H128(x[r] * su)) (su from record
// (0, kb), src/exl3-ggml.cpp:60-73), rows padded with zeros to the tile height,
// stored in MFMA A-fragment order so that the GEMM loads one fragment as one
// contiguous kilobyte: block (rows 32 rb .. +31, k 128 kb + 16 ks .. +15) is 64
// lanes x 8 halves, lane l = row % 32 + 32 (k % 16 / 8), element k % 8; blocks
// ordered (rb, kb, ks), so (rb, kb) is one contiguous 8 KB run.
__host__ __device__ inline size_t gemm_xh_offset(int row, int kb, int e, int kbs) {  // halves
    const int ks = e >> 4, kk = e & 15;
    const int ln = (row & 31) + 32 * (kk >> 3);
    return ((((size_t)(row >> 5) * kbs + kb) * 8 + ks) * 64 + ln) * 8 + (kk & 7);
}
// Workgroup (kb, rb), 4 waves x 8 rows (two passes of 4); lane 16 g + l holds
// elements 8 i .. 8 i + 7, i = h128_lane_block(l), of row 32 rb + 8 wave + 4 pass
// + g.  H128 stages 1, 2 and 4 are inside the lane, 8 .. 64 pair it with the
// lanes holding i ^ 1 .. 8 (one DPP read each); the lane's eight results are one
// 16-byte unit of the fragment layout, stored directly.
template <bool XF16>
__device__ __forceinline__ void xprep_load(const void *__restrict__ x, const size_t (&off)[2], float (&v)[2][8]) {
#pragma unroll
    for (int ps = 0; ps < 2; ++ps) {
        if constexpr (XF16) {
            const uint16_t *p = (const uint16_t *)x + off[ps];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[ps][j] = half_bits_to_float(p[j]);
        } else {
            const float *p = (const float *)x + off[ps];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[ps][j] = p[j];
        }
    }
}
__global__ __launch_bounds__(256) void gemm_xprep_kernel(const uint8_t *__restrict__ records, int bits,
                                                         const void *__restrict__ x, int x_f16, size_t x_stride,
                                                         int rows, int kbs, uint16_t *__restrict__ xh16) {
    // i: this lane's 8-element block of the row (h128_lane_block order)
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 4, i = h128_lane_block(lane & 15);
    const int kb = blockIdx.x, rb = blockIdx.y;
    const size_t col = (size_t)kb * 128 + 8 * i;
    const uint4 su8 = *(const uint4 *)(records + (size_t)kb * group_bytes(bits) + 2048 * bits + 16 * i);
    const uint32_t suw[4] = {su8.x, su8.y, su8.z, su8.w};
    float v[2][8];
    size_t off[2];  // rows past the end read row 0
#pragma unroll
    for (int ps = 0; ps < 2; ++ps) {
        const int r = 32 * rb + 8 * wave + 4 * ps + g;
        off[ps] = (size_t)(r < rows ? r : 0) * x_stride + col;
    }
    if (x_f16) xprep_load<true>(x, off, v);  // all loads before the first use
    else xprep_load<false>(x, off, v);
    // stage-major over the 16 values of both passes: independent DPP reads and
    // butterflies back to back, no wait states between a write and its DPP read
#pragma unroll
    for (int ps = 0; ps < 2; ++ps) {
        const int r = 32 * rb + 8 * wave + 4 * ps + g;
#pragma unroll
        for (int j = 0; j < 8; ++j)
            v[ps][j] = r < rows ? v[ps][j] * half_bits_to_float((uint16_t)(suw[j >> 1] >> (16 * (j & 1)))) : 0.f;
    }
#pragma unroll
    for (int st = 1; st < 8; st <<= 1)
#pragma unroll
        for (int ps = 0; ps < 2; ++ps)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (!(j & st)) {
                    const float a = v[ps][j], b = v[ps][j | st];
                    v[ps][j] = a + b;
                    v[ps][j | st] = a - b;
                }
    auto lane_stage = [&](auto sc) {
        constexpr int S = decltype(sc)::value;
        const float sgn = (i & S) ? -1.f : 1.f;
        float p[2][8];
#pragma unroll
        for (int ps = 0; ps < 2; ++ps)
#pragma unroll
            for (int j = 0; j < 8; ++j) p[ps][j] = dpp_block_xor<S>(v[ps][j]);
#pragma unroll
        for (int ps = 0; ps < 2; ++ps)
#pragma unroll
            for (int j = 0; j < 8; ++j) v[ps][j] = __builtin_fmaf(v[ps][j], sgn, p[ps][j]);
    };
    lane_stage(std::integral_constant<int, 1>{});
    lane_stage(std::integral_constant<int, 2>{});
    lane_stage(std::integral_constant<int, 4>{});
    lane_stage(std::integral_constant<int, 8>{});
#pragma unroll
    for (int ps = 0; ps < 2; ++ps) {
        const int r = 32 * rb + 8 * wave + 4 * ps + g;
        float e[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) e[j] = v[ps][j] * 0.08838834764831844055f;
        uint4 out;
        out.x = (uint32_t)float_to_half_bits(e[0]) | ((uint32_t)float_to_half_bits(e[1]) << 16);
        out.y = (uint32_t)float_to_half_bits(e[2]) | ((uint32_t)float_to_half_bits(e[3]) << 16);
        out.z = (uint32_t)float_to_half_bits(e[4]) | ((uint32_t)float_to_half_bits(e[5]) << 16);
        out.w = (uint32_t)float_to_half_bits(e[6]) | ((uint32_t)float_to_half_bits(e[7]) << 16);
        *(uint4 *)(xh16 + gemm_xh_offset(r, kb, 8 * i, kbs)) = out;
    }
}

// GEMM (rows > 32).  Workgroup (split s, m-tile mt, column group nb): rows
// [BM mt, +BM) x columns [128 nb, +128), records kb in [kb0, kb1); BM = 64 RB
// rows, wave w owning rows 32 RB w .. +32 RB for all 128 columns: RB x 4
// accumulator blocks of v_mfma_f32_32x32x16_f16 (one wave per SIMD keeps this
// MFMA at full rate; the 16x16 one needs two).  Per record kb, software-pipelined
// in straight-line code per k-step (16 k):
//   * MFMAs of k-step ks (A = activations, B = decoded weights), the B fragments
//     of k-step ks + 1 already being read from LDS;
//   * one eighth of the decode of record kb + 1 (fragment ks / 2 of the wave's
//     chunk ks % 2: the GEMV's chunk decoder) into the other LDS buffer W[n][k]
//     (fp16, 16-byte k-chunks XOR-swizzled by n % 16: conflict-free MFMA B
//     reads), interleaved with the MFMAs;
//   * the activations of k-step ks of record kb + 1 (xh16, fragment-tiled and
//     L2-resident: every column group reads it), into the registers just consumed.
// The weight words are loaded two records ahead.  MFMA 32x32x16 operands: A lane l
// = row l % 32, k 8 (l / 32) + j; B lane l = column l % 32, k 8 (l / 32) + j;
// D element e of lane l = row (e % 4) + 8 (e / 4) + 4 (l / 32), column l % 32.
// Split-K partials (kept in the accumulator layout) are summed in split order by
// the last workgroup of the tile, which applies H128 over the 128 columns of
// each row in registers (strides 1..16: lanes, 32 and 64: blocks) and sv
// (src/exl3-ggml.cpp:84-90).
constexpr int kGemmTargetWgs = 256;  // one 4-wave workgroup per CU (the accumulators fill the register file)

__device__ __forceinline__ int gemm_w_offset(int n, int chunk) {  // halves
    return n * 128 + ((chunk ^ (n & 15)) << 3);
}


// Output of accumulator values in the 32x32 MFMA D layout: t[cb][i] is column
// 32 cb + lane % 32 of row row0 + (i % 4) + 8 (i / 4) + 4 (lane / 32).  H128 over
// the 128 columns of each row in natural stage order (strides 1..16 pair lanes
// lane ^ 1..16 by DPP and v_permlane16_swap, strides 32 and 64 pair blocks cb ^ 1, 2;
// src/exl3_codec.cpp:153-165),
// then 1/sqrt(128) and sv (src/exl3-ggml.cpp:84-90).
template <int NE>
__device__ __forceinline__ void gemm_rows_out(float (&t)[4][NE], int lane, int row0, const uint16_t *svp, int rows,
                                              void *y, int y_f16, size_t y_stride, size_t col0, const void *res,
                                              size_t res_stride) {
    const int l32 = lane & 31, lh = lane >> 5;
    // lane stages stage-major over the 4 NE independent values: the DPP reads
    // and butterflies of one stage issue back to back without wait states
    auto lane_stage = [&](auto sc) {
        constexpr int S = decltype(sc)::value;
        if constexpr (S == 16) {  // v_permlane16_swap (lane_butterfly): VALU, no LDS round trip
#pragma unroll
            for (int cb = 0; cb < 4; ++cb)
#pragma unroll
                for (int i = 0; i < NE; ++i) t[cb][i] = lane_butterfly<16>(t[cb][i], l32);
        } else {
            const float sgn = (l32 & S) ? -1.f : 1.f;
            float p[4][NE];
#pragma unroll
            for (int cb = 0; cb < 4; ++cb)
#pragma unroll
                for (int i = 0; i < NE; ++i) p[cb][i] = dpp_xor<S>(t[cb][i]);
#pragma unroll
            for (int cb = 0; cb < 4; ++cb)
#pragma unroll
                for (int i = 0; i < NE; ++i) t[cb][i] = __builtin_fmaf(t[cb][i], sgn, p[cb][i]);
        }
    };
    lane_stage(std::integral_constant<int, 1>{});
    lane_stage(std::integral_constant<int, 2>{});
    lane_stage(std::integral_constant<int, 4>{});
    lane_stage(std::integral_constant<int, 8>{});
    lane_stage(std::integral_constant<int, 16>{});
#pragma unroll
    for (int st = 1; st < 4; st <<= 1)
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
            if (!(cb & st))
#pragma unroll
                for (int i = 0; i < NE; ++i) {
                    const float a = t[cb][i], b = t[cb | st][i];
                    t[cb][i] = a + b;
                    t[cb | st][i] = a - b;
                }
    float svv[4];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) svv[cb] = half_bits_to_float(svp[32 * cb + l32]);
    // res (y's dtype): y = res + layer with one rounding of the sum
    auto store = [&](auto is_f16, auto has_res) {
        constexpr bool YF16 = decltype(is_f16)::value, RES = decltype(has_res)::value;
        typedef typename std::conditional<YF16, uint16_t, float>::type T;
#pragma unroll
        for (int i = 0; i < NE; ++i) {
            const int row = row0 + (i & 3) + 8 * (i >> 2) + 4 * lh;
            if (row < rows) {
                T *yr = (T *)y + (size_t)row * y_stride + col0 + l32;
                const T *rr = (const T *)res + (size_t)row * res_stride + col0 + l32;
#pragma unroll
                for (int cb = 0; cb < 4; ++cb) {
                    float v = t[cb][i] * 0.08838834764831844055f * svv[cb];
                    if constexpr (RES) {
                        if constexpr (YF16) v += half_bits_to_float(rr[32 * cb]);
                        else v += rr[32 * cb];
                    }
                    if constexpr (YF16) yr[32 * cb] = float_to_half_bits(v);
                    else yr[32 * cb] = v;
                }
            }
        }
    };
    if (res) {
        if (y_f16) store(std::true_type{}, std::true_type{});
        else store(std::false_type{}, std::true_type{});
    } else {
        if (y_f16) store(std::true_type{}, std::false_type{});
        else store(std::false_type{}, std::false_type{});
    }
}

template <int K, int CB, int RB>
__global__ __launch_bounds__(kGemmWaves * 64) void gemm_kernel(
    const uint8_t *__restrict__ records, int kbs, int nbs, int mtiles, int splits, int kq, int kr,
    const uint16_t *__restrict__ xh16, size_t k, uint16_t *__restrict__ partials, void *y, int y_f16, size_t y_stride,
    int rows, const void *res, size_t res_stride) {
    constexpr int BM = 32 * RB * kGemmWaves;
    constexpr size_t GB = (size_t)2048 * K + 512;
    __shared__ __attribute__((aligned(16))) uint16_t wlds[2][128 * 128];  // 64 KB

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lg = lane >> 4, li = lane & 15, j = li & 7;
    const int l32 = lane & 31, lh = lane >> 5;
    // Workgroups are dispatched to the 8 XCDs round-robin (blockIdx % 8) and each
    // XCD has its own L2: renumber so that XCD x runs the contiguous range
    // [x G / 8, (x + 1) G / 8) of the order (split, column group, m-tile), m-tile
    // fastest.  The m-tiles of one column group then share its weight records,
    // and the column groups of one split share its activation rows, in one L2.
    const int G = gridDim.x;
    int L = (G & 7) ? (int)blockIdx.x : (int)(blockIdx.x & 7) * (G >> 3) + (int)(blockIdx.x >> 3);
    const int s = L / (mtiles * nbs);
    L -= s * mtiles * nbs;
    const int nb = L / mtiles, mt = L - nb * mtiles;
    const int tile = mt * nbs + nb;
    // split s owns kq + (s < kr) records from kb0 (kq = kbs / splits, kr = kbs % splits, from the host)
    const int kb0 = s * kq + (s < kr ? s : kr), kb1 = kb0 + kq + (s < kr ? 1 : 0);
    const uint8_t *colgroup = records + (size_t)nb * kbs * GB;

    // weights: this wave decodes groups q = 2 wave + h (h = 0, 1) of every record
    uint32_t wlane[2];
    int wn0[2], wc0[2];  // column and k-chunk of fragment 0 of each chunk
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int q = 2 * wave + h, r4 = q >> 2, c2 = q & 3;
        wlane[h] = (uint32_t)(r4 * 1024 * K + ((8 * lg + 2 * c2 + (li >> 3)) * 32 + 4 * j) * K);
        wn0[h] = 16 * (2 * c2 + (li >> 3)) + j;
        wc0[h] = 2 * (4 * r4 + lg);
    }
    auto load_words = [&](int kb, uint32_t (&w)[2][K]) {
        const uint8_t *rec = colgroup + (size_t)(kb < kb1 ? kb : kb1 - 1) * GB;  // past the end: re-read, unused
        load_chunk<K>(rec + wlane[0], w[0]);
        load_chunk<K>(rec + wlane[1], w[1]);
    };
    const bool first_chunk = j == 0;
    // boundary words of the two chunks (see decode_chunk), for the pieces below
    auto chunk_prepare = [&](const uint32_t (&w)[2][K], uint32_t (&xb)[2][K]) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t p1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)w[h][K - 1], 0x121, 0xF, 0xF, false);
            const uint32_t p9 = (uint32_t)__builtin_amdgcn_mov_dpp((int)w[h][K - 1], 0x129, 0xF, 0xF, false);
            xb[h][0] = __builtin_amdgcn_alignbit(first_chunk ? p9 : p1, w[h][0], 16);
#pragma unroll
            for (int m = 1; m < K; ++m) xb[h][m] = __builtin_amdgcn_alignbit(w[h][m - 1], w[h][m], 16);
        }
    };
    // piece P: fragment F = P / 2 of chunk h = P % 2 -> LDS at column
    // n0 + 8 (F >> 1), k-chunk c0 + (F & 1)
    auto decode_piece = [&](auto pc, const uint32_t (&w)[2][K], const uint32_t (&xb)[2][K], uint16_t *dst) {
        constexpr int F = decltype(pc)::value >> 1, h = decltype(pc)::value & 1;
        const u4 fr = chunk_frag<K, CB, F>(w[h], xb[h]);
        *(u4 *)(dst + gemm_w_offset(wn0[h] + 8 * (F >> 1), wc0[h] + (F & 1))) = fr;
    };
    // activations: A fragment (ks, rb) = the contiguous kilobyte of row block
    // (BM mt + 32 (RB wave + rb)) / 32, record kb, k-step ks (gemm_xh_offset)
    const uint16_t *xblk = xh16 + ((size_t)(mt * BM / 32 + RB * wave) * kbs * 8 * 64 + lane) * 8;
    auto load_x_step = [&](int kb, int ks, h8 (&xs)[RB]) {
        const uint16_t *p = xblk + ((size_t)(kb < kb1 ? kb : kb1 - 1) * 8 + ks) * 512;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) xs[rb] = *(const h8 *)(p + (size_t)rb * kbs * 8 * 512);
    };
    // B fragment (ks, cb): column 32 cb + l32, k-chunk 2 ks + lh; the swizzle term
    // depends on the lane and k-step only, so the four blocks sit at constant
    // offsets from one address
    auto read_b = [&](const uint16_t *wsrc, int ks, h8 (&b)[4]) {
        const uint16_t *base = wsrc + l32 * 128 + (((2 * ks + lh) ^ li) << 3);
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) b[cb] = *(const h8 *)(base + cb * 32 * 128);
    };

    f16v acc[RB][4];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[rb][cb][e] = 0.f;
    auto mma_step = [&](const h8 (&xs)[RB], const h8 (&b)[4]) {
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
                acc[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xs[rb], b[cb], acc[rb][cb], 0, 0, 0);
    };

    // prologue: words of kb0 and kb0 + 1, activations of kb0, record kb0 decoded,
    // B fragments of its first k-step
    uint32_t wbuf[2][2][K], xb[2][K];
    h8 xa[8][RB];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) load_x_step(kb0, ks, xa[ks]);
    load_words(kb0, wbuf[0]);
    load_words(kb0 + 1, wbuf[1]);
    chunk_prepare(wbuf[0], xb);
    decode_piece(std::integral_constant<int, 0>{}, wbuf[0], xb, wlds[0]);
    decode_piece(std::integral_constant<int, 1>{}, wbuf[0], xb, wlds[0]);
    decode_piece(std::integral_constant<int, 2>{}, wbuf[0], xb, wlds[0]);
    decode_piece(std::integral_constant<int, 3>{}, wbuf[0], xb, wlds[0]);
    decode_piece(std::integral_constant<int, 4>{}, wbuf[0], xb, wlds[0]);
    decode_piece(std::integral_constant<int, 5>{}, wbuf[0], xb, wlds[0]);
    decode_piece(std::integral_constant<int, 6>{}, wbuf[0], xb, wlds[0]);
    decode_piece(std::integral_constant<int, 7>{}, wbuf[0], xb, wlds[0]);
    __syncthreads();
    h8 bc[4], bn[4];
    read_b(wlds[0], 0, bc);

    // one k-step: B of ks + 1 requested, MFMAs of ks, a decode piece, then the
    // activations of ks for the next record
    auto kstep = [&](auto kc, int kb, const uint16_t *wcur, uint16_t *wnext, const uint32_t (&wnextw)[2][K],
                     h8 (&bcur)[4], h8 (&bnxt)[4]) {
        constexpr int KS = decltype(kc)::value;
        if constexpr (KS < 7) read_b(wcur, KS + 1, bnxt);
        mma_step(xa[KS], bcur);
        decode_piece(std::integral_constant<int, KS>{}, wnextw, xb, wnext);
        load_x_step(kb + 1, KS, xa[KS]);
        // One MFMA every few VALU instructions: the wave issues in order, so
        // MFMAs back to back stall it while the decode waits behind them.  The
        // B reads lead, the activation loads (seven k-steps ahead of their use:
        // left alone the scheduler sinks them to the end of the record) trail.
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            if (i < 4) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
            __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);  // VALU
            if (i == 7) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // LDS write
            if (i >= 6) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // global load
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // record kb: activations xa, decoded weights wcur (B fragments of k-step 0 in
    // bc); words of kb + 1 in wnextw; slot wfree takes the words of kb + 2
    auto step = [&](int kb, const uint16_t *wcur, uint16_t *wnext, uint32_t (&wfree)[2][K],
                    const uint32_t (&wnextw)[2][K]) {
        load_words(kb + 2, wfree);
        chunk_prepare(wnextw, xb);
        kstep(std::integral_constant<int, 0>{}, kb, wcur, wnext, wnextw, bc, bn);
        kstep(std::integral_constant<int, 1>{}, kb, wcur, wnext, wnextw, bn, bc);
        kstep(std::integral_constant<int, 2>{}, kb, wcur, wnext, wnextw, bc, bn);
        kstep(std::integral_constant<int, 3>{}, kb, wcur, wnext, wnextw, bn, bc);
        kstep(std::integral_constant<int, 4>{}, kb, wcur, wnext, wnextw, bc, bn);
        kstep(std::integral_constant<int, 5>{}, kb, wcur, wnext, wnextw, bn, bc);
        kstep(std::integral_constant<int, 6>{}, kb, wcur, wnext, wnextw, bc, bn);
        kstep(std::integral_constant<int, 7>{}, kb, wcur, wnext, wnextw, bn, bc);
        __syncthreads();  // wnext complete; every wave is done reading wcur
        read_b(wnext, 0, bc);
    };
    int kb = kb0;
    for (; kb + 2 <= kb1; kb += 2) {
        step(kb, wlds[0], wlds[1], wbuf[0], wbuf[1]);
        step(kb + 1, wlds[1], wlds[0], wbuf[1], wbuf[0]);
    }
    if (kb < kb1) {  // odd count: the last record is in wlds[0]
#pragma unroll
        for (int ks = 0; ks < 8; ks += 2) {
            read_b(wlds[0], ks + 1, bn);
            mma_step(xa[ks], bc);
            if (ks + 2 < 8) read_b(wlds[0], ks + 2, bc);
            mma_step(xa[ks + 1], bn);
        }
    }

    // epilogue.  acc[rb][cb][e]: row 32 RB wave + 32 rb + (e % 4) + 8 (e / 4) + 4 lh,
    // column 32 cb + l32
    if (splits > 1) {
        // fp16 partials in accumulator layout [tile][split][wave][rb][cb][vp][lane]
        // x 16 bytes: elements 8 vp .. 8 vp + 7 of acc[rb][cb] (rows of v = 2 vp,
        // 2 vp + 1), summed in fp32 by gemm_reduce_kernel.  fp16 keeps the layer
        // within its tolerance (rel-L2 2.9e-4 against 2.1e-4 for fp32 partials
        // with fp16 output, at k = 14336) for half the bytes.
        constexpr size_t kPerSplit = (size_t)kGemmWaves * RB * 4 * 2 * 64 * 8;  // halves
        uint16_t *dst = partials + ((size_t)tile * splits + s) * kPerSplit + (size_t)wave * RB * 8 * 512 + lane * 8;
        auto pk = [](float a, float b) {
            return (uint32_t)float_to_half_bits(a) | ((uint32_t)float_to_half_bits(b) << 16);
        };
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int cb = 0; cb < 4; ++cb)
#pragma unroll
                for (int vp = 0; vp < 2; ++vp) {
                    const f16v &a = acc[rb][cb];
                    const u4 d = {pk(a[8 * vp], a[8 * vp + 1]), pk(a[8 * vp + 2], a[8 * vp + 3]),
                                  pk(a[8 * vp + 4], a[8 * vp + 5]), pk(a[8 * vp + 6], a[8 * vp + 7])};
                    __builtin_nontemporal_store(d, (u4 *)(dst + ((rb * 4 + cb) * 2 + vp) * 512));
                }
        return;
    }
    const uint16_t *svp = (const uint16_t *)(colgroup + 2048 * K + 256);  // record (nb, 0)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        float t[4][16];
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
#pragma unroll
            for (int e = 0; e < 16; ++e) t[cb][e] = acc[rb][cb][e];
        gemm_rows_out<16>(t, lane, mt * BM + 32 * RB * wave + 32 * rb, svp, rows, y, y_f16, y_stride, (size_t)nb * 128,
                          res, res_stride);
    }
}

// Split-K reduction (split count > 1): one wave per (tile, row block blk =
// RB wave + rb, vp) of the GEMM's partial layout; lane l sums its 4 x 16 bytes
// (fp16) of every split in fp32 in split order (so the result does not depend on
// the order the GEMM's workgroups ran in), then H128, 1/sqrt(128) and sv over its
// 16 rows.
template <int RB>
__global__ __launch_bounds__(256) void gemm_reduce_kernel(const uint16_t *__restrict__ partials, int splits, int nbs,
                                                          const uint8_t *__restrict__ records, int bits, int kbs,
                                                          void *y, int y_f16, size_t y_stride, int rows,
                                                          int nwaves, const void *res, size_t res_stride) {
    constexpr int BM = 32 * RB * kGemmWaves;
    constexpr size_t kPerSplit = (size_t)kGemmWaves * RB * 4 * 2 * 64 * 8;  // halves
    const int lane = threadIdx.x & 63;
    const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (gw >= nwaves) return;
    const int vp = gw & 1, blk = (gw >> 1) % (kGemmWaves * RB), tile = (gw >> 1) / (kGemmWaves * RB);
    const int mt = tile / nbs, nb = tile - mt * nbs;
    const uint16_t *src = partials + (size_t)tile * splits * kPerSplit + (size_t)blk * 8 * 512 + vp * 512 + lane * 8;
    float t[4][8];
#pragma unroll 1
    for (int sp0 = 0; sp0 < splits; sp0 += 4) {  // loads of four splits in flight, then their sum in order
        u4 in[4][4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int sp = sp0 + u < splits ? sp0 + u : splits - 1;
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) in[u][cb] = *(const u4 *)(src + (size_t)sp * kPerSplit + cb * 2 * 512);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (sp0 + u < splits)
#pragma unroll
                for (int cb = 0; cb < 4; ++cb) {
                    const uint32_t w[4] = {in[u][cb].x, in[u][cb].y, in[u][cb].z, in[u][cb].w};
#pragma unroll
                    for (int q = 0; q < 8; ++q) {
                        const float v = half_bits_to_float((uint16_t)(w[q >> 1] >> (16 * (q & 1))));
                        t[cb][q] = sp0 + u == 0 ? v : t[cb][q] + v;
                    }
                }
    }
    const uint16_t *svp = (const uint16_t *)(records + (size_t)nb * kbs * group_bytes(bits) + 2048 * bits + 256);
    gemm_rows_out<8>(t, lane, mt * BM + 32 * blk + 16 * vp, svp, rows, y, y_f16, y_stride, (size_t)nb * 128, res,
                     res_stride);
}

int gemm_tile_rows(size_t rows) { return rows <= 128 ? 128 : 256; }

GemmPlan gemm_plan(size_t k, size_t n, size_t rows) {
    GemmPlan p{};
    p.nbs = (int)(n / 128);
    p.kbs = (int)(k / 128);
    p.bm = gemm_tile_rows(rows);
    p.mtiles = (int)((rows + p.bm - 1) / p.bm);
    const int tiles = p.nbs * p.mtiles;
    // split k only below kGemmSplitTiles tiles; the split partials are summed by
    // gemm_reduce_kernel
    int s = tiles >= (int)kGemmSplitTiles ? 1 : (kGemmTargetWgs + tiles - 1) / tiles;
    const int smax = p.kbs / 4 > 0 ? p.kbs / 4 : 1;
    s = s < 1 ? 1 : (s > smax ? smax : s);
    p.splits = s;
    size_t off = 0;
    p.counters_off = off;
    off += counter_region_bytes(n);
    p.xh_off = off;
    off += ((size_t)p.mtiles * p.bm * k * 2 + 255) & ~(size_t)255;
    p.partials_off = off;
    if (s > 1) off += (size_t)tiles * s * p.bm * 128 * 2;  // fp16 partials
    p.bytes = (off + 255) & ~(size_t)255;
    return p;
}

template <int K, int CB>
static void launch_gemm_kc(const uint8_t *rec, size_t k, uint16_t *xh, size_t rows, void *y, int y_f16,
                           size_t y_stride, uint8_t *ws, const GemmPlan &p, hipStream_t stream, const void *res,
                           size_t res_stride) {
    const dim3 grid((unsigned)(p.mtiles * p.nbs * p.splits)), block(kGemmWaves * 64);
    uint16_t *part = (uint16_t *)(ws + p.partials_off);
    const int nwaves = p.mtiles * p.nbs * (p.bm / 16);  // reduction: one wave per 16 rows of a tile
    const int kq = p.kbs / p.splits, kr = p.kbs % p.splits;
    const dim3 rgrid((unsigned)((nwaves + 3) / 4));
    if (p.bm == 128) {
        gemm_kernel<K, CB, 1><<<grid, block, 0, stream>>>(rec, p.kbs, p.nbs, p.mtiles, p.splits, kq, kr, xh, k, part,
                                                          y, y_f16, y_stride, (int)rows, res, res_stride);
        if (p.splits > 1)
            gemm_reduce_kernel<1><<<rgrid, dim3(256), 0, stream>>>(part, p.splits, p.nbs, rec, K, p.kbs, y, y_f16,
                                                                   y_stride, (int)rows, nwaves, res, res_stride);
    } else {
        gemm_kernel<K, CB, 2><<<grid, block, 0, stream>>>(rec, p.kbs, p.nbs, p.mtiles, p.splits, kq, kr, xh, k, part,
                                                          y, y_f16, y_stride, (int)rows, res, res_stride);
        if (p.splits > 1)
            gemm_reduce_kernel<2><<<rgrid, dim3(256), 0, stream>>>(part, p.splits, p.nbs, rec, K, p.kbs, y, y_f16,
                                                                   y_stride, (int)rows, nwaves, res, res_stride);
    }
}

template <int K>
static hipError_t launch_gemm_k(const void *records, int cb, size_t k, const void *x, int x_f16, size_t rows,
                                size_t x_stride, void *y, int y_f16, size_t y_stride, uint8_t *ws, const GemmPlan &p,
                                hipStream_t stream, const void *res, size_t res_stride) {
    const uint8_t *rec = (const uint8_t *)records;
    uint16_t *xh = (uint16_t *)(ws + p.xh_off);
    const int rows_padded = p.mtiles * p.bm;
    gemm_xprep_kernel<<<dim3(p.kbs, rows_padded / 32), dim3(256), 0, stream>>>(rec, K, x, x_f16, x_stride, (int)rows,
                                                                               p.kbs, xh);
    switch (cb) {
    case 0: launch_gemm_kc<K, 0>(rec, k, xh, rows, y, y_f16, y_stride, ws, p, stream, res, res_stride); break;
    case 1: launch_gemm_kc<K, 1>(rec, k, xh, rows, y, y_f16, y_stride, ws, p, stream, res, res_stride); break;
    default: launch_gemm_kc<K, 2>(rec, k, xh, rows, y, y_f16, y_stride, ws, p, stream, res, res_stride); break;
    }
    return hipGetLastError();
}

hipError_t launch_gemm(const void *records, int bits, int cb, size_t k, size_t n, const void *x, int x_f16,
                       size_t rows, size_t x_stride, void *y, int y_f16, size_t y_stride, void *workspace,
                       const GemmPlan &p, hipStream_t stream, const void *res, size_t res_stride) {
    (void)n;
    uint8_t *ws = (uint8_t *)workspace;
    switch (bits) {
    case 1: return launch_gemm_k<1>(records, cb, k, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream, res,
                                       res_stride);
    case 2: return launch_gemm_k<2>(records, cb, k, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream, res,
                                       res_stride);
    case 3: return launch_gemm_k<3>(records, cb, k, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream, res,
                                       res_stride);
    case 4: return launch_gemm_k<4>(records, cb, k, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream, res,
                                       res_stride);
    case 5: return launch_gemm_k<5>(records, cb, k, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream, res,
                                       res_stride);
    case 6: return launch_gemm_k<6>(records, cb, k, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream, res,
                                       res_stride);
    case 7: return launch_gemm_k<7>(records, cb, k, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream, res,
                                       res_stride);
    default: return launch_gemm_k<8>(records, cb, k, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream, res,
                                       res_stride);
    }
}

}  // namespace exl3k
