// exl3_codec_kernels.hip -- gfx950 codec kernels of the EXL3 layer:
//   codebook_kernel    exl3::decode_codebook, bit-exact
//   hadamard_kernel    exl3::hadamard128, bit-exact
//   decode_kernel      trellis tiles -> row-major fp16, bit-exact (exl3::decode_inner);
//   decode_batch_kernel the same for many whole matrices per launch
//   reconstruct_kernel original-basis weights, bit-exact (exl3::reconstruct)
//   get_rows_kernel    GET_ROWS: columns of the original-basis weights (ggml_exl3_get_rows)
//   pack_records_kernel, validate_kernel, zero_kernel
// Reference semantics: src/exl3_codec.cpp, src/exl3-ggml.cpp:19-49.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "exl3_kernel_common.hpp"

namespace exl3k {

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
// kDecodeBlocksPerWg consecutive blocks b (bx, rk) = (b % gx, b / gx), gx =
// ceil(n / 256), from b = kDecodeBlocksPerWg (w - wg_begin[m]): a tile row's
// neighbouring 256-column blocks.  The next block's stream words are loaded
// while the current one is decoded, transposed (two LDS buffers) and stored, so
// a workgroup keeps a block's loads in flight behind its stores.
template <int K>
__device__ __forceinline__ bool decode_block_load(const uint8_t *__restrict__ src, int records_layout, size_t k,
                                                  size_t n, size_t tile_count, size_t gx, size_t b,
                                                  uint32_t (&w)[RunGeo<K>::NW]) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t bx = b % gx, rk = b / gx, t0 = bx * 16;
    const int tl = wave * 4 + (lane >> 4);
    const int c = lane & 7, h = (lane >> 3) & 1;
    if (t0 + tl >= tile_count) return false;
    load_run_words<K>(tile_ptr<K>(src, records_layout, k, n, rk, t0 + tl), c, h, w);
    return true;
}

template <int K, int CB>
__device__ __forceinline__ void decode_block_store(const uint32_t (&w)[RunGeo<K>::NW], bool valid, size_t tile_count,
                                                   size_t gx, size_t b, uint16_t *__restrict__ out, uint16_t *tb) {
    constexpr int PITCH = kDecodePitch;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t bx = b % gx, rk = b / gx, t0 = bx * 16;
    const int tl = wave * 4 + (lane >> 4);
    const int c = lane & 7, h = (lane >> 3) & 1;
    if (valid) {
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
        const int ch = tid + 256 * i;  // 16 rows x 32 chunks of 8 halves
        const int row = ch >> 5, col8 = ch & 31;
        const int tl2 = col8 >> 1;
        if (t0 + tl2 < tile_count) {
            const u4 v = *(const u4 *)(tb + row * PITCH + col8 * 8);
            __builtin_nontemporal_store(v, (u4 *)(out + (rk * 16 + row) * count + (t0 + tl2) * 16 + (col8 & 1) * 8));
        }
    }
}

template <int K, int CB>
__global__ __launch_bounds__(256) void decode_batch_kernel(DecodeBatch batch, int records_layout) {
    __shared__ uint16_t tb[2][16 * kDecodePitch];  // one block's transpose while the other's is read
    const unsigned w = blockIdx.x;
    int m = 0;
    for (int i = 1; i < batch.count; ++i)
        if (w >= batch.wg_begin[i]) m = i;
    const size_t k = batch.k[m], n = batch.n[m];
    const size_t tiles = n / 16, gx = (tiles + 15) / 16, nblk = (k / 16) * gx;
    const size_t b0 = (size_t)(w - batch.wg_begin[m]) * kDecodeBlocksPerWg;
    const uint8_t *src = (const uint8_t *)batch.src[m];
    uint32_t wa[RunGeo<K>::NW], wb[RunGeo<K>::NW];
    bool va = decode_block_load<K>(src, records_layout, k, n, tiles, gx, b0, wa), vb = false;
#pragma unroll
    for (int j = 0; j < kDecodeBlocksPerWg; j += 2) {  // two register sets: no copy of words in flight
        if (b0 + j >= nblk) break;  // uniform
        if (b0 + j + 1 < nblk) vb = decode_block_load<K>(src, records_layout, k, n, tiles, gx, b0 + j + 1, wb);
        decode_block_store<K, CB>(wa, va, tiles, gx, b0 + j, batch.out[m], tb[0]);
        if (b0 + j + 1 >= nblk) break;
        if (j + 2 < kDecodeBlocksPerWg && b0 + j + 2 < nblk)
            va = decode_block_load<K>(src, records_layout, k, n, tiles, gx, b0 + j + 2, wa);
        decode_block_store<K, CB>(wb, vb, tiles, gx, b0 + j + 1, batch.out[m], tb[1]);
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
                                                       const int32_t *__restrict__ ids, size_t ids_stride,
                                                       void *__restrict__ out, int out_f16, size_t out_stride,
                                                       int *__restrict__ bad_ids) {
    constexpr int P = 129;
    __shared__ float blk[128 * P];
    __shared__ float colv[128];
    const int tid = threadIdx.x;
    const size_t r = blockIdx.x, kb = blockIdx.y;
    const int32_t id = ids[r * ids_stride];
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
static hipError_t launch_get_rows_k(const void *records, int cb, size_t k, size_t n, const int32_t *ids,
                                    size_t ids_stride, size_t count, void *out, int out_f16, size_t out_stride,
                                    int *bad_ids, hipStream_t stream) {
    const dim3 grid((unsigned)count, (unsigned)(k / 128)), block(256);
    const uint8_t *rec = (const uint8_t *)records;
    switch (cb) {
    case 0: get_rows_kernel<K, 0><<<grid, block, 0, stream>>>(rec, k, n, ids, ids_stride, out, out_f16, out_stride,
                                                                 bad_ids); break;
    case 1: get_rows_kernel<K, 1><<<grid, block, 0, stream>>>(rec, k, n, ids, ids_stride, out, out_f16, out_stride,
                                                                 bad_ids); break;
    default: get_rows_kernel<K, 2><<<grid, block, 0, stream>>>(rec, k, n, ids, ids_stride, out, out_f16, out_stride,
                                                                 bad_ids); break;
    }
    return hipGetLastError();
}

hipError_t launch_get_rows(const void *records, int bits, int cb, size_t k, size_t n, const int32_t *ids,
                           size_t ids_stride, size_t count, void *out, int out_f16, size_t out_stride, int *bad_ids,
                           hipStream_t stream) {
    switch (bits) {
    case 1: return launch_get_rows_k<1>(records, cb, k, n, ids, ids_stride, count, out, out_f16, out_stride, bad_ids, stream);
    case 2: return launch_get_rows_k<2>(records, cb, k, n, ids, ids_stride, count, out, out_f16, out_stride, bad_ids, stream);
    case 3: return launch_get_rows_k<3>(records, cb, k, n, ids, ids_stride, count, out, out_f16, out_stride, bad_ids, stream);
    case 4: return launch_get_rows_k<4>(records, cb, k, n, ids, ids_stride, count, out, out_f16, out_stride, bad_ids, stream);
    case 5: return launch_get_rows_k<5>(records, cb, k, n, ids, ids_stride, count, out, out_f16, out_stride, bad_ids, stream);
    case 6: return launch_get_rows_k<6>(records, cb, k, n, ids, ids_stride, count, out, out_f16, out_stride, bad_ids, stream);
    case 7: return launch_get_rows_k<7>(records, cb, k, n, ids, ids_stride, count, out, out_f16, out_stride, bad_ids, stream);
    default: return launch_get_rows_k<8>(records, cb, k, n, ids, ids_stride, count, out, out_f16, out_stride, bad_ids, stream);
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

}  // namespace exl3k
