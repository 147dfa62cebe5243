// exl3_kernels.hip -- gfx950 kernels of the EXL3 packed-weight linear layer.
//
//   gemv_kernel      rows 1..8: each lane decodes 16 trellis positions of a tile
//                    straight into an fp16 MFMA A-fragment (W^T), the activations
//                    H128(x*su) arrive pre-split into fp16 hi/lo halves in the 16
//                    MFMA columns, v_mfma_f32_16x16x32_f16 accumulates in fp32;
//                    split-K partials are reduced in fixed order by the last
//                    workgroup of each 128-column group, which applies H128 and sv.
//   gemm_kernel      rows > 8: a workgroup decodes one 128x128 record per step into
//                    LDS (fp16, n-major), streams a 128-row activation tile through
//                    LDS and runs 16x16x32 f16 MFMAs, fp32 accumulation.
//   decode_kernel    trellis tiles -> row-major fp16, bit-exact (exl3::decode_inner).
//   reconstruct_kernel original-basis weights, bit-exact (exl3::reconstruct).
// Reference semantics: src/exl3_codec.cpp, src/exl3-ggml.cpp:51-92.
#include <hip/hip_runtime.h>
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
// One workgroup: one 16-row tile row rk, 16 consecutive tile columns.
// Lane (wave w, lane l): tile w*4 + l/16, run c = l%8, h = (l%16)/8.
template <int K, int CB>
__global__ __launch_bounds__(256) void decode_kernel(const uint8_t *__restrict__ src, int records_layout, size_t k,
                                                     size_t n, size_t first_tile, size_t tile_count,
                                                     uint16_t *__restrict__ out) {
    constexpr int PITCH = 16 * 16 + 8;
    __shared__ uint16_t tb[16 * PITCH];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t rk = blockIdx.y;
    const size_t t0 = (size_t)blockIdx.x * 16;  // first tile (relative to first_tile) of this workgroup
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
            const uint4 v = *(const uint4 *)(tb + row * PITCH + col8 * 8);
            *(uint4 *)(out + (rk * 16 + row) * count + (t0 + tl2) * 16 + (col8 & 1) * 8) = v;
        }
    }
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
// One launch per call.  Workgroup (nb, split s) owns slabs [u0, u1) (32 input rows
// each) of the 128-column group nb and walks them in chunks of kChunk slabs:
//   1. prep: xh[r] = H128(x[r] * su) in fp32 for the 128-row blocks the chunk
//      touches (su from record (0, kb), src/exl3-ggml.cpp:60-73), split into fp16
//      hi = rn(xh), lo = rn(xh - hi) and scattered into MFMA B fragments in LDS:
//      slab u, lane = m + 16 g, element j; column m < 8 holds hi of row m,
//      column m >= 8 holds lo of row m - 8 (zero for absent rows);
//   2. wave w takes slabs u0 + w, u0 + w + 4, ...; per slab a lane decodes, for
//      each tile-column pair tp, one run of tile (k-tile 2 (u % 4) + g / 2,
//      n-tile 2 tp + nl / 8), c = nl % 8, h = g % 2 (nl = lane % 16, g = lane / 16)
//      and issues two MFMAs (A = decoded W^T fragment, B = activations).  The
//      next slab's words are loaded while the current one is decoded.
// D^T[n][m]: lane l holds m = l % 16, n_local = 4 (l / 16) + e.  Split-K
// partials are reduced in fixed order by the last workgroup of the column group,
// which also applies H128 and sv (src/exl3-ggml.cpp:84-90).
// Weight stream of a wave: a slab is 2 k-tiles x 8 n-tiles (512 K contiguous bytes
// of a record); each lane loads the NLOAD words of its 4 runs straight into
// registers, DEPTH slabs ahead (statically unrolled so every wait the compiler
// inserts is exact).
template <int K>
struct GemvStream {
    static constexpr int SLAB = 512 * K;
    static constexpr int WORDS = 4 * RunGeo<K>::NLOAD;                   // registers per slab and lane
    static constexpr int DEPTH = WORDS <= 12 ? 4 : (WORDS <= 16 ? 3 : 2);
};
constexpr int kFusedPrepRows = 2;    // rows <= this: activation prep inside the GEMV kernel
constexpr int kMaxPrepBlocks = 4;    // (kb, row) blocks a wave prepares in the fused path

// Four agent-coherent loads issued together, then one wait (relaxed atomic loads
// are otherwise issued one round trip at a time).
__device__ __forceinline__ float4 load4_coherent(const float *p0, const float *p1, const float *p2, const float *p3) {
    float4 r;
    asm volatile(
        "global_load_dword %0, %4, off sc1\n\t"
        "global_load_dword %1, %5, off sc1\n\t"
        "global_load_dword %2, %6, off sc1\n\t"
        "global_load_dword %3, %7, off sc1\n\t"
        "s_waitcnt vmcnt(0)"
        : "=&v"(r.x), "=&v"(r.y), "=&v"(r.z), "=&v"(r.w)
        : "v"(p0), "v"(p1), "v"(p2), "v"(p3)
        : "memory");
    return r;
}

// Compact B-fragment layout of a slab (128 * rows bytes): 16-byte groups
// ((hl * rows + r) * 4 + g), hl = 0 hi / 1 lo, r = row, g = lane / 16; element j of
// a group is k row 16 (g / 2) + R_{g % 2}(j) of the slab.  Lane l of the MFMA
// B operand reads group (hl, r, g) with m = l % 16 -> (hl, r) = (m / 8, m % 8), or
// a zero group when r >= rows.
__device__ __forceinline__ int frag_elem_offset(int rho32, int hl, int r, int rows) {
    const int kt = rho32 >> 4, r16 = rho32 & 15;
    const int hh = (r16 >> 2) & 1;
    const int j = (r16 & 1) | (((r16 >> 3) & 1) << 1) | (((r16 >> 1) & 1) << 2);
    const int g = 2 * kt + hh;
    return (((hl * rows + r) * 4 + g) * 8 + j) * 2;  // bytes
}

// Write hi/lo halves of one prepared activation (row r, k row rho32 of slab ul)
__device__ __forceinline__ void frag_put(uint8_t *frag, int slab_bytes, int ul, int rho32, int r, int rows, float xv) {
    const _Float16 h16 = (_Float16)xv;
    uint8_t *base = frag + (size_t)ul * slab_bytes;
    *(uint16_t *)(base + frag_elem_offset(rho32, 0, r, rows)) = bitcast<uint16_t>(h16);
    *(uint16_t *)(base + frag_elem_offset(rho32, 1, r, rows)) = bitcast<uint16_t>((_Float16)(xv - (float)h16));
}

// hi half at p, lo half at p + lo_off (fragment byte offsets from frag_elem_offset)
__device__ __forceinline__ void frag_put2(uint8_t *p, int lo_off, float xv) {
    const _Float16 h16 = (_Float16)xv;
    *(uint16_t *)p = bitcast<uint16_t>(h16);
    *(uint16_t *)(p + lo_off) = bitcast<uint16_t>((_Float16)(xv - (float)h16));
}

// Activation prep kernel for rows > kFusedPrepRows: one workgroup (64 threads =
// one wave) per (128-row block kb, row r); writes the compact fragments of the
// four slabs of block kb.  xh = H128(x[r] * su), su from record (0, kb)
// (src/exl3-ggml.cpp:60-73).
__global__ __launch_bounds__(64) void gemv_frag_kernel(const uint8_t *__restrict__ records, int bits,
                                                       const void *__restrict__ x, int x_f16, size_t x_stride,
                                                       int rows, uint8_t *__restrict__ frag) {
    const int kb = blockIdx.x, r = blockIdx.y, lane = threadIdx.x;
    const uint16_t *su = (const uint16_t *)(records + (size_t)kb * group_bytes(bits) + 2048 * bits);
    float v0 = load_x(x, x_f16, x_stride, r, (size_t)kb * 128 + lane) * half_bits_to_float(su[lane]);
    float v1 = load_x(x, x_f16, x_stride, r, (size_t)kb * 128 + lane + 64) * half_bits_to_float(su[lane + 64]);
    h128_wave(v0, v1, lane);
    const int slab_bytes = 128 * rows;
    frag_put(frag, slab_bytes, kb * 4 + (lane >> 5), lane & 31, r, rows, v0);
    frag_put(frag, slab_bytes, kb * 4 + 2 + (lane >> 5), lane & 31, r, rows, v1);
}

// GEMV.  Workgroup (nb, split s) owns slabs [u0, u1) of the 128-column group nb;
// wave w takes slabs u0 + w, u0 + w + 4, ... and streams them through its LDS
// ring (DEPTH slabs in flight).  Per slab a lane decodes, for each tile-column
// pair tp, one run of tile (k-tile 2 (u % 4) + g / 2, n-tile 2 tp + nl / 8) with
// c = nl % 8, h = g % 2 (nl = lane % 16, g = lane / 16) and issues two MFMAs
// (A = decoded W^T fragment, B = activation fragment).  D^T[n][m]: lane l holds
// m = l % 16, n_local = 4 (l / 16) + e.  Split-K partials are reduced in fixed
// order by the last workgroup of the column group, which applies H128 and sv
// (src/exl3-ggml.cpp:84-90).
template <int K, int CB, bool FUSED>
__global__ __launch_bounds__(kGemvWaves * 64) void gemv_kernel(
    const uint8_t *__restrict__ records, int kbs, int nbs, int splits, int units, const void *__restrict__ x,
    int x_f16, size_t x_stride, int rows, const uint8_t *__restrict__ frag_global, const uint8_t *__restrict__ dummy,
    float *__restrict__ partials, unsigned *__restrict__ counters, void *__restrict__ y, int y_f16, size_t y_stride) {
    using ST = GemvStream<K>;
    constexpr int NT = kGemvWaves * 64;
    constexpr size_t GB = (size_t)2048 * K + 512;
    constexpr int NW = RunGeo<K>::NW;
    constexpr int NL = RunGeo<K>::NLOAD;
    constexpr int D = ST::DEPTH;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ int last_flag;
    uint8_t *zero16 = smem;            // 16 zero bytes: B fragment of absent rows
    uint8_t *frag = smem + 16;
    const int slab_bytes = 128 * rows;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int s = blockIdx.x / nbs, nb = blockIdx.x - s * nbs;
    const int u0 = (int)((long long)units * s / splits), u1 = (int)((long long)units * (s + 1) / splits);
    const int nl = lane & 15, g = lane >> 4;
    const int c = nl & 7, h = g & 1, ktp = g >> 1;
    const uint8_t *colgroup = records + (size_t)nb * kbs * GB;

    // 1. activation inputs (issued first: their waits never cover the weight stream)
    const int kb_first = u0 >> 2, kb_last = (u1 - 1) >> 2;
    const int nkb = kb_last - kb_first + 1;
    const int nblk = nkb * rows;
    // raw bits only: converting here would make the compiler wait for these loads
    // before the weight stream is issued
    uint32_t px0[FUSED ? kMaxPrepBlocks : 1], px1[FUSED ? kMaxPrepBlocks : 1];
    uint16_t ps0[FUSED ? kMaxPrepBlocks : 1], ps1[FUSED ? kMaxPrepBlocks : 1];
    if constexpr (FUSED) {
        // branch-free so that every load is in flight at once: blocks past nblk
        // re-read block 0 and are discarded (fused path: rows is 1 or 2)
        auto prep_loads = [&](auto is_f16) {
            constexpr bool XF16 = decltype(is_f16)::value;
#pragma unroll
            for (int q = 0; q < kMaxPrepBlocks; ++q) {
                const int blk = wave + q * kGemvWaves;
                const int bc = blk < nblk ? blk : 0;
                const int kb = kb_first + (rows == 1 ? bc : bc >> 1), r = rows == 1 ? 0 : (bc & 1);
                const uint16_t *su = (const uint16_t *)(records + (size_t)kb * GB + 2048 * K);  // record (0, kb)
                const size_t xi = (size_t)r * x_stride + (size_t)kb * 128 + lane;
                if constexpr (XF16) {
                    px0[q] = ((const uint16_t *)x)[xi];
                    px1[q] = ((const uint16_t *)x)[xi + 64];
                } else {
                    px0[q] = ((const uint32_t *)x)[xi];
                    px1[q] = ((const uint32_t *)x)[xi + 64];
                }
                ps0[q] = su[lane];
                ps1[q] = su[lane + 64];
            }
        };
        if (x_f16) prep_loads(std::true_type{});
        else prep_loads(std::false_type{});
    }
    // output scales for the epilogue (record (nb, 0), src/exl3-ggml.cpp:84-85)
    const uint16_t *svp = (const uint16_t *)(colgroup + 2048 * K + 256);
    const float sv0 = half_bits_to_float(svp[lane]), sv1 = half_bits_to_float(svp[lane + 64]);

    // 2. weight stream: this wave's slabs u0 + wave + 4 i, i < nw; DEPTH slabs in flight
    uint32_t off[NL];
    run_word_offsets<K>(c, h, off);
#pragma unroll
    for (int j = 0; j < NL; ++j) off[j] += (uint32_t)((8 * ktp + (nl >> 3)) * 32 * K);
    const int first_u = u0 + wave;
    const int nw = first_u < u1 ? (u1 - first_u + kGemvWaves - 1) / kGemvWaves : 0;
    // wave-uniform slab address: record kb = u / 4, k-tile pair 2 (u % 4); slabs past
    // the end read a zero region of the workspace, so every issue is unconditional
    // and the compiler's wait counts stay exact
    auto slab_src = [&](int i) {
        const int u = first_u + i * kGemvWaves;
        return i < nw ? colgroup + (size_t)(u >> 2) * GB + (size_t)(u & 3) * ST::SLAB : dummy;
    };
    uint32_t buf[D][4][NL];
    auto issue = [&](int i, uint32_t (&dst)[4][NL]) {
        const uint8_t *src = slab_src(i);
#pragma unroll
        for (int tp = 0; tp < 4; ++tp)
#pragma unroll
            for (int j = 0; j < NL; ++j)
                dst[tp][j] = __builtin_nontemporal_load((const uint32_t *)(src + off[j] + 2 * tp * 32 * K));
    };
#pragma unroll
    for (int d = 0; d < D; ++d) issue(d, buf[d]);

    // 3. activation fragments of slabs [u0, u1) into LDS
    if (tid < 4) ((uint32_t *)zero16)[tid] = 0u;
    if constexpr (FUSED) {
        const int lane_frag_off = frag_elem_offset(lane & 31, 0, 0, rows);
#pragma unroll
        for (int q = 0; q < kMaxPrepBlocks; ++q) {
            const int blk = wave + q * kGemvWaves;
            if (blk < nblk) {
                const int kb = kb_first + (rows == 1 ? blk : blk >> 1), r = rows == 1 ? 0 : (blk & 1);
                const float xa = x_f16 ? half_bits_to_float((uint16_t)px0[q]) : bitcast<float>(px0[q]);
                const float xb = x_f16 ? half_bits_to_float((uint16_t)px1[q]) : bitcast<float>(px1[q]);
                float v0 = xa * half_bits_to_float(ps0[q]), v1 = xb * half_bits_to_float(ps1[q]);
                h128_wave(v0, v1, lane);
                const int ua = kb * 4 + (lane >> 5), ub = kb * 4 + 2 + (lane >> 5);
                const int eo = lane_frag_off + r * 64;   // + hl * rows * 64 for the lo half
                if (ua >= u0 && ua < u1) frag_put2(frag + (size_t)(ua - u0) * slab_bytes + eo, rows * 64, v0);
                if (ub >= u0 && ub < u1) frag_put2(frag + (size_t)(ub - u0) * slab_bytes + eo, rows * 64, v1);
            }
        }
    } else {
        const uint4 *src = (const uint4 *)(frag_global + (size_t)u0 * slab_bytes);
        uint4 *dst = (uint4 *)frag;
        for (int t = tid; t < (u1 - u0) * slab_bytes / 16; t += NT) dst[t] = src[t];
    }
    __syncthreads();

    // 4. decode + MFMA
    const int mrow = nl & 7, mhl = nl >> 3;
    const bool bvalid = mrow < rows;
    const int boff = bvalid ? ((mhl * rows + mrow) * 4 + g) * 16 : 0;
    const uint8_t *bbase = bvalid ? frag : zero16;
    const int bstride = bvalid ? slab_bytes : 0;
    f4 acc[4][2];
#pragma unroll
    for (int tp = 0; tp < 4; ++tp) acc[tp][0] = acc[tp][1] = (f4){0.f, 0.f, 0.f, 0.f};
    // words of slab i -> run windows (registers), then refill buf with slab i + D, then decode
    auto take = [&](int i, const uint32_t (&src)[4][NL], uint32_t (&w)[4][NW]) {
#pragma unroll
        for (int tp = 0; tp < 4; ++tp) {
            if constexpr (RunGeo<K>::ODD) {
                const uint32_t sh = h ? 16u : 0u;
#pragma unroll
                for (int j = 0; j < NW; ++j) w[tp][j] = __builtin_amdgcn_alignbit(src[tp][j], src[tp][j + 1], sh);
            } else {
#pragma unroll
                for (int j = 0; j < NW; ++j) w[tp][j] = src[tp][j];
            }
        }
        (void)i;
    };
    auto mac = [&](int i, const uint32_t (&w)[4][NW]) {
        const int u = first_u + i * kGemvWaves;
        const h8 b = *(const h8 *)(bbase + (size_t)(u - u0) * bstride + boff);
#pragma unroll
        for (int tp = 0; tp < 4; ++tp) {
            u4 a1, a2;
            decode_run<K, CB>(w[tp], a1, a2);
            acc[tp][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bitcast<h8>(a1), b, acc[tp][0], 0, 0, 0);
            acc[tp][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bitcast<h8>(a2), b, acc[tp][1], 0, 0, 0);
        }
    };
    int i0 = 0;
    for (; i0 + D <= nw; i0 += D) {  // full groups: no branches between issue and use
#pragma unroll
        for (int d = 0; d < D; ++d) {
            uint32_t w[4][NW];
            take(i0 + d, buf[d], w);
            issue(i0 + d + D, buf[d]);   // words are in registers; refill the slot
            mac(i0 + d, w);
        }
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {  // tail: fewer than D slabs, already in flight
        if (i0 + d < nw) {
            uint32_t w[4][NW];
            take(i0 + d, buf[d], w);
            mac(i0 + d, w);
        }
    }

    // 5. epilogue: hi + lo (MFMA column m < 8 gets column m + 8), then the wave sum in LDS
    __syncthreads();  // every wave is done with the fragments; LDS now holds the wave partials
    float *red = (float *)smem;
#pragma unroll
    for (int tp = 0; tp < 4; ++tp)
#pragma unroll
        for (int mf = 0; mf < 2; ++mf)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float v = acc[tp][mf][e];
                // row_shl:8 -> lane m of each 16-lane row reads lane m + 8 (the lo half)
                const float o = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x108, 0xF, 0xF, true));
                if (nl < rows && nl < 8) {
                    const int nloc = 4 * g + e;
                    const int col = 16 * (2 * tp + (nloc >> 3)) + (nloc & 7) + 8 * mf;
                    red[(wave * kGemvMaxRows + nl) * 128 + col] = v + o;
                }
            }
    __syncthreads();
    constexpr int PER = kGemvMaxRows * 128 / NT;
    float part[PER];
    const int nval = rows * 128;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int t = tid + i * NT;
        float sum = 0.f;
        if (t < nval) {
            const int rr = t >> 7, col = t & 127;
#pragma unroll
            for (int wv = 0; wv < kGemvWaves; ++wv) sum += red[(wv * kGemvMaxRows + rr) * 128 + col];
        }
        part[i] = sum;
    }
    if (splits > 1) {
        float *mine = partials + ((size_t)nb * splits + s) * (size_t)nval;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int t = tid + i * NT;
            if (t < nval) store_coherent(mine + t, part[i]);
        }
        if (!arrive_last(counters + nb, (unsigned)splits, &last_flag)) return;
        const float *all = partials + (size_t)nb * splits * (size_t)nval;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int t = tid + i * NT;
            float sum = 0.f;
            if (t < nval) {
                const float *q = all + t;
                int sp = 0;
                for (; sp + 4 <= splits; sp += 4) {
                    const float4 f = load4_coherent(q + (size_t)sp * nval, q + (size_t)(sp + 1) * nval,
                                                    q + (size_t)(sp + 2) * nval, q + (size_t)(sp + 3) * nval);
                    sum += f.x;
                    sum += f.y;
                    sum += f.z;
                    sum += f.w;
                }
                for (; sp < splits; ++sp) sum += load_coherent(q + (size_t)sp * nval);
            }
            part[i] = sum;
        }
        if (tid == 0) reset_counter(counters + nb);  // self-reset for the next call
    }
    // 6. output H128 per row (one wave per row, registers) and sv
    float *ybuf = red + kGemvWaves * kGemvMaxRows * 128;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int t = tid + i * NT;
        if (t < nval) ybuf[t] = part[i];
    }
    __syncthreads();
    for (int rr = wave; rr < rows; rr += kGemvWaves) {
        float a0 = ybuf[rr * 128 + lane], a1 = ybuf[rr * 128 + lane + 64];
        h128_wave(a0, a1, lane);
        a0 *= sv0;
        a1 *= sv1;
        const size_t o = (size_t)rr * y_stride + (size_t)nb * 128;
        if (y_f16) {
            ((uint16_t *)y)[o + lane] = float_to_half_bits(a0);
            ((uint16_t *)y)[o + lane + 64] = float_to_half_bits(a1);
        } else {
            ((float *)y)[o + lane] = a0;
            ((float *)y)[o + lane + 64] = a1;
        }
    }
}

GemvPlan gemv_plan(size_t k, size_t n, size_t rows) {
    GemvPlan p{};
    p.nbs = (int)(n / 128);
    p.kbs = (int)(k / 128);
    p.units = (int)(k / 32);
    const bool fused = rows <= (size_t)kFusedPrepRows;
    int s = (512 + p.nbs - 1) / (p.nbs > 0 ? p.nbs : 1);
    const int smax = p.units / 4 > 0 ? p.units / 4 : 1;
    s = s < 1 ? 1 : (s > smax ? smax : s);
    // fused prep: a wave prepares at most kMaxPrepBlocks (kb, row) blocks;
    // fragments of a workgroup must fit next to the ring in LDS
    for (;;) {
        const int uwg = (p.units + s - 1) / s;
        const int nkb = (uwg + 3) / 4 + 1;
        const bool ok_prep = !fused || nkb * (int)rows <= kMaxPrepBlocks * kGemvWaves;
        const bool ok_lds = (size_t)uwg * 128 * rows <= 49152;
        if ((ok_prep && ok_lds) || s >= smax) break;
        ++s;
    }
    p.splits = s;
    size_t off = 0;
    p.counters_off = off;
    off += counter_region_bytes(n);
    p.dummy_off = off;  // 4 KB target of the stream's issues past the last slab (loaded, never used)
    off += 4096;
    p.xprep_off = off;  // compact activation fragments (prep-kernel path)
    if (!fused) off += ((size_t)p.units * 128 * rows + 255) & ~(size_t)255;
    p.partials_off = off;
    if (s > 1) off += (size_t)p.nbs * s * rows * 128 * 4;
    p.bytes = (off + 255) & ~(size_t)255;
    return p;
}

template <int K, int CB>
static hipError_t launch_gemv_kc(const uint8_t *rec, const void *x, int x_f16, size_t rows, size_t x_stride, void *y,
                                 int y_f16, size_t y_stride, uint8_t *ws, const GemvPlan &p, hipStream_t stream) {
    const bool fused = rows <= (size_t)kFusedPrepRows;
    const int uwg = (p.units + p.splits - 1) / p.splits;
    const size_t frag_bytes = 16 + (size_t)uwg * 128 * rows;
    const size_t red_bytes = (size_t)kGemvWaves * kGemvMaxRows * 128 * 4 + (size_t)kGemvMaxRows * 128 * 4;
    size_t lds = frag_bytes > red_bytes ? frag_bytes : red_bytes;
    lds = (lds + 15) & ~(size_t)15;
    const dim3 grid((unsigned)(p.nbs * p.splits)), block(kGemvWaves * 64);
    float *part = (float *)(ws + p.partials_off);
    unsigned *cnt = (unsigned *)(ws + p.counters_off);
    uint8_t *frag = ws + p.xprep_off;
    const uint8_t *dummy = ws + p.dummy_off;
    if (fused) {
        gemv_kernel<K, CB, true><<<grid, block, lds, stream>>>(rec, p.kbs, p.nbs, p.splits, p.units, x, x_f16, x_stride,
                                                               (int)rows, nullptr, dummy, part, cnt, y, y_f16, y_stride);
    } else {
        gemv_frag_kernel<<<dim3(p.kbs, (unsigned)rows), dim3(64), 0, stream>>>(rec, K, x, x_f16, x_stride, (int)rows, frag);
        gemv_kernel<K, CB, false><<<grid, block, lds, stream>>>(rec, p.kbs, p.nbs, p.splits, p.units, x, x_f16,
                                                                x_stride, (int)rows, frag, dummy, part, cnt, y, y_f16, y_stride);
    }
    return hipGetLastError();
}

template <int K>
static hipError_t launch_gemv_k(const void *records, int cb, const void *x, int x_f16, size_t rows, size_t x_stride,
                                void *y, int y_f16, size_t y_stride, uint8_t *ws, const GemvPlan &p,
                                hipStream_t stream) {
    const uint8_t *rec = (const uint8_t *)records;
    switch (cb) {
    case 0: return launch_gemv_kc<K, 0>(rec, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream);
    case 1: return launch_gemv_kc<K, 1>(rec, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream);
    default: return launch_gemv_kc<K, 2>(rec, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream);
    }
}

hipError_t launch_gemv(const void *records, int bits, int cb, size_t k, size_t n, const void *x, int x_f16,
                       size_t rows, size_t x_stride, void *y, int y_f16, size_t y_stride, void *workspace,
                       const GemvPlan &p, hipStream_t stream) {
    (void)k;
    (void)n;
    uint8_t *ws = (uint8_t *)workspace;
    switch (bits) {
    case 1: return launch_gemv_k<1>(records, cb, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream);
    case 2: return launch_gemv_k<2>(records, cb, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream);
    case 3: return launch_gemv_k<3>(records, cb, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream);
    case 4: return launch_gemv_k<4>(records, cb, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream);
    case 5: return launch_gemv_k<5>(records, cb, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream);
    case 6: return launch_gemv_k<6>(records, cb, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream);
    case 7: return launch_gemv_k<7>(records, cb, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream);
    default: return launch_gemv_k<8>(records, cb, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream);
    }
}

// ============================================================== GEMM
// Activation prep for the GEMM: xh16[r][i] = fp16(H128(x[r] * su)[i]), rows padded
// to a multiple of 128 with zeros.  Grid (kbs, mtiles*16), 128 threads, 8 rows each.
__global__ __launch_bounds__(128) void gemm_xprep_kernel(const uint8_t *__restrict__ records, int bits,
                                                         const void *__restrict__ x, int x_f16, size_t x_stride,
                                                         int rows, size_t k, uint16_t *__restrict__ xh16) {
    __shared__ float v[8 * 129];
    const int kb = blockIdx.x, t = threadIdx.x, r0 = blockIdx.y * 8;
    const uint16_t *su = (const uint16_t *)(records + (size_t)kb * group_bytes(bits) + 2048 * bits);
    const float s = half_bits_to_float(su[t]);
    for (int r = 0; r < 8; ++r)
        v[r * 129 + t] = (r0 + r < rows) ? load_x(x, x_f16, x_stride, r0 + r, (size_t)kb * 128 + t) * s : 0.f;
    __syncthreads();
    h128_lds(v, 8, 129, t, 128);
    for (int r = 0; r < 8; ++r) xh16[(size_t)(r0 + r) * k + (size_t)kb * 128 + t] = float_to_half_bits(v[r * 129 + t]);
}

// Workgroup (m-tile mt, column group nb, split s): rows [128 mt, +128) x columns
// [128 nb, +128), records kb in [kb0, kb1).  4 waves in a 2 x 2 grid, each
// 64 x 64 = 4 x 4 MFMA blocks.  Per record: x tile -> LDS (row-major), record
// decoded -> LDS n-major (Ws[n][k]), 4 k-steps of 16x16x32 MFMAs.
template <int K, int CB>
__global__ __launch_bounds__(kGemmWaves * 64) void gemm_kernel(
    const uint8_t *__restrict__ records, int kbs, int nbs, int mtiles, int splits, const uint16_t *__restrict__ xh16,
    size_t k, float *__restrict__ partials, unsigned *__restrict__ counters, void *__restrict__ y, int y_f16,
    size_t y_stride, int rows) {
    constexpr int NT = kGemmWaves * 64;
    constexpr int XP = 128 + 8;   // LDS pitch (halves) of the activation and weight tiles
    constexpr int OP = 128 + 4;   // LDS pitch (floats) of the output tile
    constexpr size_t GB = (size_t)2048 * K + 512;
    constexpr int LDS_BYTES = (2 * 128 * XP * 2) > (128 * OP * 4) ? (2 * 128 * XP * 2) : (128 * OP * 4);
    __shared__ __attribute__((aligned(16))) uint8_t smem[LDS_BYTES];
    __shared__ int last_flag;
    uint16_t *Xs = (uint16_t *)smem;
    uint16_t *Ws = Xs + 128 * XP;
    float *Os = (float *)smem;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    int bid = blockIdx.x;
    const int s = bid % splits;
    bid /= splits;
    const int nb = bid % nbs, mt = bid / nbs;
    const int kb0 = (int)((long long)kbs * s / splits), kb1 = (int)((long long)kbs * (s + 1) / splits);

    f4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = (f4){0.f, 0.f, 0.f, 0.f};

    const uint16_t *xbase = xh16 + (size_t)mt * 128 * k;
    for (int kb = kb0; kb < kb1; ++kb) {
        // activation tile 128 x 128 fp16: 2048 uint4, 8 per thread
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int ch = tid + i * NT;
            const int row = ch >> 4, c8 = ch & 15;
            *(uint4 *)(Xs + row * XP + c8 * 8) = *(const uint4 *)(xbase + (size_t)row * k + (size_t)kb * 128 + c8 * 8);
        }
        // decode the record: 1024 runs, 4 per thread, into Ws[n][k]
        const uint8_t *rec = records + ((size_t)nb * kbs + kb) * GB;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int run = tid + i * NT;
            const int tile = run >> 4, rc = run & 15;
            const int c = rc & 7, h = rc >> 3, tr = tile >> 3, tc = tile & 7;
            uint32_t w[RunGeo<K>::NW];
            load_run_words<K>((const uint32_t *)(rec + (8 * tr + tc) * 32 * K), c, h, w);
            u4 a1, a2;
            decode_run<K, CB>(w, a1, a2);
            const uint32_t p1[4] = {a1.x, a1.y, a1.z, a1.w}, p2[4] = {a2.x, a2.y, a2.z, a2.w};
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int kr = tr * 16 + run_slot_row(h, 2 * v);  // even row; pair = rows kr, kr + 1
                *(uint32_t *)(Ws + (tc * 16 + c) * XP + kr) = p1[v];
                *(uint32_t *)(Ws + (tc * 16 + c + 8) * XP + kr) = p2[v];
            }
        }
        __syncthreads();
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            h8 a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                a[i] = *(const h8 *)(Xs + (wm * 64 + i * 16 + (lane & 15)) * XP + ks * 32 + 8 * (lane >> 4));
#pragma unroll
            for (int j = 0; j < 4; ++j)
                b[j] = *(const h8 *)(Ws + (wn * 64 + j * 16 + (lane & 15)) * XP + ks * 32 + 8 * (lane >> 4));
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }
    // D[m][n]: lane l holds n = l % 16, m = 4 (l / 16) + e
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                Os[(wm * 64 + i * 16 + 4 * (lane >> 4) + e) * OP + wn * 64 + j * 16 + (lane & 15)] = acc[i][j][e];
    __syncthreads();
    const int row0 = mt * 128;
    const int vrows = rows - row0 < 128 ? rows - row0 : 128;
    if (splits > 1) {
        float *mine = partials + (((size_t)mt * nbs + nb) * splits + s) * 128 * 128;
        for (int t = tid; t < vrows * 128; t += NT) store_coherent(mine + t, Os[(t >> 7) * OP + (t & 127)]);
        if (!arrive_last(counters + (size_t)mt * nbs + nb, (unsigned)splits, &last_flag)) return;
        const float *all = partials + ((size_t)mt * nbs + nb) * splits * 128 * 128;
        for (int t = tid; t < vrows * 128; t += NT) {
            float sum = 0.f;
            for (int sp = 0; sp < splits; ++sp) sum += load_coherent(all + (size_t)sp * 128 * 128 + t);
            Os[(t >> 7) * OP + (t & 127)] = sum;
        }
        if (tid == 0) reset_counter(counters + (size_t)mt * nbs + nb);
        __syncthreads();
    }
    h128_lds(Os, vrows, OP, tid, NT);
    const uint16_t *sv = (const uint16_t *)(records + (size_t)nb * kbs * GB + 2048 * K + 256);
    for (int t = tid; t < vrows * 128; t += NT) {
        const int rr = t >> 7, col = t & 127;
        const float v = Os[rr * OP + col] * half_bits_to_float(sv[col]);
        const size_t o = (size_t)(row0 + rr) * y_stride + (size_t)nb * 128 + col;
        if (y_f16) ((uint16_t *)y)[o] = float_to_half_bits(v);
        else ((float *)y)[o] = v;
    }
}

GemmPlan gemm_plan(size_t k, size_t n, size_t rows) {
    GemmPlan p{};
    p.nbs = (int)(n / 128);
    p.kbs = (int)(k / 128);
    p.mtiles = (int)((rows + 127) / 128);
    const int tiles = p.nbs * p.mtiles;
    // split k only below kGemmSplitTiles tiles (then s == 1): counters stay in their region
    int s = tiles >= (int)kGemmSplitTiles ? 1 : ((int)kGemmSplitTiles + tiles - 1) / tiles;
    const int smax = p.kbs / 4 > 0 ? p.kbs / 4 : 1;
    s = s < 1 ? 1 : (s > smax ? smax : s);
    p.splits = s;
    size_t off = 0;
    p.counters_off = off;
    off += counter_region_bytes(n);
    p.xh_off = off;
    off += (size_t)p.mtiles * 128 * k * 2;
    p.partials_off = off;
    if (s > 1) off += (size_t)tiles * s * 128 * 128 * 4;
    p.bytes = (off + 255) & ~(size_t)255;
    return p;
}

template <int K>
static hipError_t launch_gemm_k(const void *records, int cb, size_t k, const void *x, int x_f16, size_t rows,
                                size_t x_stride, void *y, int y_f16, size_t y_stride, uint8_t *ws, const GemmPlan &p,
                                hipStream_t stream) {
    const uint8_t *rec = (const uint8_t *)records;
    uint16_t *xh = (uint16_t *)(ws + p.xh_off);
    gemm_xprep_kernel<<<dim3(p.kbs, p.mtiles * 16), dim3(128), 0, stream>>>(rec, K, x, x_f16, x_stride, (int)rows, k, xh);
    const dim3 grid((unsigned)(p.mtiles * p.nbs * p.splits)), block(kGemmWaves * 64);
    float *part = (float *)(ws + p.partials_off);
    unsigned *cnt = (unsigned *)(ws + p.counters_off);
    switch (cb) {
    case 0: gemm_kernel<K, 0><<<grid, block, 0, stream>>>(rec, p.kbs, p.nbs, p.mtiles, p.splits, xh, k, part, cnt, y, y_f16, y_stride, (int)rows); break;
    case 1: gemm_kernel<K, 1><<<grid, block, 0, stream>>>(rec, p.kbs, p.nbs, p.mtiles, p.splits, xh, k, part, cnt, y, y_f16, y_stride, (int)rows); break;
    default: gemm_kernel<K, 2><<<grid, block, 0, stream>>>(rec, p.kbs, p.nbs, p.mtiles, p.splits, xh, k, part, cnt, y, y_f16, y_stride, (int)rows); break;
    }
    return hipGetLastError();
}

hipError_t launch_gemm(const void *records, int bits, int cb, size_t k, size_t n, const void *x, int x_f16,
                       size_t rows, size_t x_stride, void *y, int y_f16, size_t y_stride, void *workspace,
                       const GemmPlan &p, hipStream_t stream) {
    (void)n;
    uint8_t *ws = (uint8_t *)workspace;
    switch (bits) {
    case 1: return launch_gemm_k<1>(records, cb, k, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream);
    case 2: return launch_gemm_k<2>(records, cb, k, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream);
    case 3: return launch_gemm_k<3>(records, cb, k, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream);
    case 4: return launch_gemm_k<4>(records, cb, k, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream);
    case 5: return launch_gemm_k<5>(records, cb, k, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream);
    case 6: return launch_gemm_k<6>(records, cb, k, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream);
    case 7: return launch_gemm_k<7>(records, cb, k, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream);
    default: return launch_gemm_k<8>(records, cb, k, x, x_f16, rows, x_stride, y, y_f16, y_stride, ws, p, stream);
    }
}

}  // namespace exl3k
