// exl3_gemm.hip -- the EXL3 layer at rows > 32 on gfx950 (gemm_xprep_kernel,
// gemm_kernel, gemm_reduce_kernel): H128(x*su) once in fp16 MFMA-fragment order;
// a workgroup (k split, column group, m-tile) decodes record kb + 1 into LDS
// (fp16, swizzled) while v_mfma_f32_32x32x16_f16 runs on record kb, fp32
// accumulation; split partials are summed in fixed order by the reduce kernel,
// which applies H128 and sv.
// Reference semantics: src/exl3-ggml.cpp:51-92.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include <type_traits>

#include "exl3_kernel_common.hpp"

namespace exl3k {

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
// Workgroup (kb, 4 rb + wave) is one wave of 8 rows (two passes of 4; one wave
// per workgroup spreads a short prep over more CUs than 4-wave workgroups:
// -0.1 to -0.35 us per call at 24..512 rows); lane 16 g + l holds elements
// 8 i .. 8 i + 7, i = h128_lane_block(l), of row 32 rb + 8 wave + 4 pass + g.  H128 stages 1, 2 and 4 are inside the lane, 8 .. 64 pair it with the
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
__global__ __launch_bounds__(64) void gemm_xprep_kernel(const uint8_t *__restrict__ records, int bits,
                                                         const void *__restrict__ x, int x_f16, size_t x_stride,
                                                         int rows, int kbs, uint16_t *__restrict__ xh16) {
    // i: this lane's 8-element block of the row (h128_lane_block order)
    const int lane = threadIdx.x & 63, wave = blockIdx.y & 3, g = lane >> 4, i = h128_lane_block(lane & 15);
    const int kb = blockIdx.x, rb = blockIdx.y >> 2;
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
    // cross-lane stages in signed form, one DPP fmac per value (the GEMV prep's
    // dpp_block_stage8): the stage signs multiply into one lane sign, applied
    // with the 1/sqrt(128) scale; the same roundings as sgn v + v'
    auto lane_stage = [&](auto sc) {
        constexpr int S = decltype(sc)::value;
        const float sgn = (i & S) ? -1.f : 1.f;
        dpp_block_stage8<S>(v[0], sgn);
        dpp_block_stage8<S>(v[1], sgn);
    };
    lane_stage(std::integral_constant<int, 1>{});
    lane_stage(std::integral_constant<int, 2>{});
    lane_stage(std::integral_constant<int, 4>{});
    lane_stage(std::integral_constant<int, 8>{});
    const float scale = (__builtin_popcount(i & 15) & 1) ? -0.08838834764831844055f : 0.08838834764831844055f;
#pragma unroll
    for (int ps = 0; ps < 2; ++ps) {
        const int r = 32 * rb + 8 * wave + 4 * ps + g;
        float e[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) e[j] = v[ps][j] * scale;
        uint4 out;
        out.x = (uint32_t)float_to_half_bits(e[0]) | ((uint32_t)float_to_half_bits(e[1]) << 16);
        out.y = (uint32_t)float_to_half_bits(e[2]) | ((uint32_t)float_to_half_bits(e[3]) << 16);
        out.z = (uint32_t)float_to_half_bits(e[4]) | ((uint32_t)float_to_half_bits(e[5]) << 16);
        out.w = (uint32_t)float_to_half_bits(e[6]) | ((uint32_t)float_to_half_bits(e[7]) << 16);
        *(uint4 *)(xh16 + gemm_xh_offset(r, kb, 8 * i, kbs)) = out;
    }
}

// GEMM (rows > 32).  Workgroup (split s, m-tile mt, column group nb) of W waves
// (4 or 8): rows [BM mt, +BM) x columns [128 nb, +128), records kb in [kb0, kb1);
// BM = 32 RB W rows, wave w owning rows 32 RB w .. +32 RB for all 128 columns:
// RB x 4 accumulator blocks of v_mfma_f32_32x32x16_f16 (one wave per SIMD keeps
// this MFMA at full rate; the 16x16 one needs two).  Per record kb,
// software-pipelined in straight-line code per k-step (16 k):
//   * MFMAs of k-step ks (A = activations, B = decoded weights), the B fragments
//     of k-step ks + 1 already being read from LDS;
//   * a share of the decode of record kb + 1 (each wave decodes H = 8 / W of the
//     record's eight trellis chunks with the GEMV's chunk decoder, one fragment
//     per k-step or every other k-step) into the other LDS buffer W[n][k] (fp16,
//     16-byte k-chunks XOR-swizzled by n % 16: conflict-free MFMA B reads),
//     interleaved with the MFMAs;
//   * the activations of k-step ks + XD (xh16, fragment-tiled and L2-resident:
//     every column group reads it), into the registers just consumed.
// The weight words are loaded two records ahead.  MFMA 32x32x16 operands: A lane l
// = row l % 32, k 8 (l / 32) + j; B lane l = column l % 32, k 8 (l / 32) + j;
// D element e of lane l = row (e % 4) + 8 (e / 4) + 4 (l / 32), column l % 32.
// Without a k split the workgroup applies H128 over the 128 columns of each row
// in registers (strides 1..16: lanes, 32 and 64: blocks) and sv
// (src/exl3-ggml.cpp:84-90); with one, gemm_reduce_kernel sums the partials in
// split order and does the same.
constexpr int kGemmTargetWgs = 256;  // one workgroup per CU (the accumulators fill the register file)

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

// CH column parts: with CH = 2 (4) the W waves are W / CH row waves x CH column
// parts, each wave owning 32 RB rows x 128 / CH columns (4 / CH accumulator
// blocks per row block), so that a 128-row (64-row) tile runs two waves per
// SIMD and a 32-row tile four waves per workgroup; such a tile always has a k
// split (its epilogue writes partials only).
template <int K, int CB, int RB, int W, int NSG, int XD, int CH>
__global__ __launch_bounds__(W * 64) void gemm_kernel(
    const uint8_t *__restrict__ records, int kbs, int nbs, int mtiles, int splits, int kq, int kr,
    const uint16_t *__restrict__ xh16, size_t k, uint16_t *__restrict__ partials, int *__restrict__ exps, void *y,
    int y_f16, size_t y_stride, int rows, const void *res, size_t res_stride) {
    constexpr int WR = W / CH;   // waves along the rows
    constexpr int NCB = 4 / CH;  // 32-column accumulator blocks per row block of a wave
    constexpr int BM = 32 * RB * WR;
    constexpr int H = 8 / W;  // trellis chunks a wave decodes per record
    constexpr size_t GB = (size_t)2048 * K + 512;
    __shared__ __attribute__((aligned(16))) uint16_t wlds[2][128 * 128];  // 64 KB

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rw = wave % WR, ch = wave / WR;  // row wave, column half
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

    // weights: this wave decodes groups q = H wave + h (h < H) of every record
    uint32_t wlane[H];
    int wn0[H], wc0[H];  // column and k-chunk of fragment 0 of each chunk
#pragma unroll
    for (int h = 0; h < H; ++h) {
        const int q = H * wave + h, r4 = q >> 2, c2 = q & 3;
        wlane[h] = (uint32_t)(r4 * 1024 * K + ((8 * lg + 2 * c2 + (li >> 3)) * 32 + 4 * j) * K);
        wn0[h] = 16 * (2 * c2 + (li >> 3)) + j;
        wc0[h] = 2 * (4 * r4 + lg);
    }
    auto load_words = [&](int kb, uint32_t (&w)[H][K]) {
        const uint8_t *rec = colgroup + (size_t)(kb < kb1 ? kb : kb1 - 1) * GB;  // past the end: re-read, unused
#pragma unroll
        for (int h = 0; h < H; ++h) load_chunk<K>(rec + wlane[h], w[h]);
    };
    const bool first_chunk = j == 0;
    auto chunk_prepare = [&](const uint32_t (&w)[H][K], uint32_t (&xb)[H][K]) {
#pragma unroll
        for (int h = 0; h < H; ++h) {
            const uint32_t p1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)w[h][K - 1], 0x121, 0xF, 0xF, false);
            const uint32_t p9 = (uint32_t)__builtin_amdgcn_mov_dpp((int)w[h][K - 1], 0x129, 0xF, 0xF, false);
            xb[h][0] = __builtin_amdgcn_alignbit(first_chunk ? p9 : p1, w[h][0], 16);
#pragma unroll
            for (int m = 1; m < K; ++m) xb[h][m] = __builtin_amdgcn_alignbit(w[h][m - 1], w[h][m], 16);
        }
    };
    // piece P (0 .. 4 H - 1): fragment F = P / H of chunk h = P % H -> LDS at
    // column n0 + 8 (F >> 1), k-chunk c0 + (F & 1)
    auto decode_piece = [&](auto pc, const uint32_t (&w)[H][K], const uint32_t (&xb)[H][K], uint16_t *dst) {
        constexpr int F = decltype(pc)::value / H, h = decltype(pc)::value % H;
        const u4 fr = chunk_frag<K, CB, F>(w[h], xb[h]);
        *(u4 *)(dst + gemm_w_offset(wn0[h] + 8 * (F >> 1), wc0[h] + (F & 1))) = fr;
    };
    // activations: A fragment (ks, rb) = the contiguous kilobyte of row block
    // (BM mt + 32 (RB rw + rb)) / 32, record kb, k-step ks (gemm_xh_offset)
    const uint16_t *xblk = xh16 + ((size_t)(mt * BM / 32 + RB * rw) * kbs * 8 * 64 + lane) * 8;
    auto load_x_step = [&](int kb, int ks, h8 (&xs)[RB]) {
        const uint16_t *p = xblk + ((size_t)(kb < kb1 ? kb : kb1 - 1) * 8 + ks) * 512;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) xs[rb] = *(const h8 *)(p + (size_t)rb * kbs * 8 * 512);
    };
    // B fragment (ks, cb): column 32 (NCB ch + cb) + l32, k-chunk 2 ks + lh; the
    // swizzle term depends on the lane and k-step only, so the blocks sit at
    // constant offsets from one address
    auto read_b = [&](const uint16_t *wsrc, int ks, h8 (&b)[NCB]) {
        const uint16_t *base = wsrc + l32 * 128 + (((2 * ks + lh) ^ li) << 3) + NCB * ch * 32 * 128;
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) b[cb] = *(const h8 *)(base + cb * 32 * 128);
    };

    f16v acc[RB][NCB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[rb][cb][e] = 0.f;
    auto mma_step = [&](const h8 (&xs)[RB], const h8 (&b)[NCB]) {
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
                acc[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xs[rb], b[cb], acc[rb][cb], 0, 0, 0);
    };

    // prologue: words of kb0 and kb0 + 1, activations of kb0, record kb0 decoded,
    // B fragments of its first k-step
    uint32_t wbuf[2][H][K], xb[H][K];
    h8 xa[XD][RB];
#pragma unroll
    for (int ks = 0; ks < XD; ++ks) load_x_step(kb0, ks, xa[ks]);
    load_words(kb0, wbuf[0]);
    load_words(kb0 + 1, wbuf[1]);
    chunk_prepare(wbuf[0], xb);
    decode_piece(std::integral_constant<int, 0>{}, wbuf[0], xb, wlds[0]);
    decode_piece(std::integral_constant<int, 1>{}, wbuf[0], xb, wlds[0]);
    decode_piece(std::integral_constant<int, 2>{}, wbuf[0], xb, wlds[0]);
    decode_piece(std::integral_constant<int, 3>{}, wbuf[0], xb, wlds[0]);
    if constexpr (H == 2) {
        decode_piece(std::integral_constant<int, 4>{}, wbuf[0], xb, wlds[0]);
        decode_piece(std::integral_constant<int, 5>{}, wbuf[0], xb, wlds[0]);
        decode_piece(std::integral_constant<int, 6>{}, wbuf[0], xb, wlds[0]);
        decode_piece(std::integral_constant<int, 7>{}, wbuf[0], xb, wlds[0]);
    }
    __syncthreads();
    h8 bc[NCB], bn[NCB];
    read_b(wlds[0], 0, bc);

    // one k-step: B of ks + 1 requested, MFMAs of ks, a decode piece, then the
    // activations of ks for the next record
    auto kstep = [&](auto kc, int kb, const uint16_t *wcur, uint16_t *wnext, const uint32_t (&wnextw)[H][K],
                     h8 (&bcur)[NCB], h8 (&bnxt)[NCB]) {
        constexpr int KS = decltype(kc)::value;
        if constexpr (KS < 7) read_b(wcur, KS + 1, bnxt);
        mma_step(xa[KS % XD], bcur);
        if constexpr (H == 2) decode_piece(std::integral_constant<int, KS>{}, wnextw, xb, wnext);
        else if constexpr (KS % 2 == 0) decode_piece(std::integral_constant<int, KS / 2>{}, wnextw, xb, wnext);
        load_x_step(KS + XD < 8 ? kb : kb + 1, (KS + XD) % 8, xa[KS % XD]);
        // One MFMA every few VALU instructions: the wave issues in order, so
        // MFMAs back to back stall it while the decode waits behind them.  The
        // B reads lead, the activation loads (seven k-steps ahead of their use:
        // left alone the scheduler sinks them to the end of the record) trail.
#pragma unroll
        for (int i = 0; i < NSG; ++i) {
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
    auto step = [&](int kb, const uint16_t *wcur, uint16_t *wnext, uint32_t (&wfree)[H][K],
                    const uint32_t (&wnextw)[H][K]) {
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
            mma_step(xa[ks % XD], bc);
            if (ks + XD < 8) load_x_step(kb, ks + XD, xa[ks % XD]);
            if (ks + 2 < 8) read_b(wlds[0], ks + 2, bc);
            mma_step(xa[(ks + 1) % XD], bn);
            if (ks + 1 + XD < 8) load_x_step(kb, ks + 1 + XD, xa[(ks + 1) % XD]);
        }
    }

    // epilogue.  acc[rb][cb][e]: row 32 RB rw + 32 rb + (e % 4) + 8 (e / 4) + 4 lh,
    // column 32 (NCB ch + cb) + l32
    if (splits > 1) {
        // fp16 partials in accumulator layout [tile][split][rw][rb][column block][vp]
        // [lane] x 16 bytes: elements 8 vp .. 8 vp + 7 of a 32x32 block (rows of
        // v = 2 vp, 2 vp + 1), summed in fp32 by gemm_reduce_kernel.  Each 32x32
        // block is stored scaled by 2^-e, e = exps[(tile, split, rw, rb, block)]
        // chosen so that its largest magnitude is below 2^14: fp16's relative
        // precision for every value, and no overflow however large the activations.
        // fp16 keeps the layer within its tolerance (rel-L2 2.9e-4 against 2.1e-4
        // for fp32 partials with fp16 output, at k = 14336) for half the bytes.
        constexpr size_t kPerSplit = (size_t)WR * RB * 4 * 2 * 64 * 8;  // halves
        uint16_t *dst = partials + ((size_t)tile * splits + s) * kPerSplit + (size_t)rw * RB * 8 * 512 + lane * 8;
        auto pk = [](float a, float b, int e) {
            return (uint32_t)float_to_half_bits(__builtin_amdgcn_ldexpf(a, -e)) |
                   ((uint32_t)float_to_half_bits(__builtin_amdgcn_ldexpf(b, -e)) << 16);
        };
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb) {
                const int cg = NCB * ch + cb;  // column block in the tile
                float m = 0.f;
#pragma unroll
                for (int e = 0; e < 16; ++e) m = fmaxf(m, fabsf(acc[rb][cb][e]));
                m = wave_max(m);
                const int ex = __builtin_amdgcn_frexp_expf(m) - 14;  // m < 2^(ex + 14); 0 (and Inf, NaN): -14
                if (lane == 0) exps[(((size_t)tile * splits + s) * (WR * RB) + rw * RB + rb) * 4 + cg] = ex;
#pragma unroll
                for (int vp = 0; vp < 2; ++vp) {
                    const f16v &a = acc[rb][cb];
                    const u4 d = {pk(a[8 * vp], a[8 * vp + 1], ex), pk(a[8 * vp + 2], a[8 * vp + 3], ex),
                                  pk(a[8 * vp + 4], a[8 * vp + 5], ex), pk(a[8 * vp + 6], a[8 * vp + 7], ex)};
                    __builtin_nontemporal_store(d, (u4 *)(dst + ((rb * 4 + cg) * 2 + vp) * 512));
                }
            }
        return;
    }
    if constexpr (CH == 1) {  // whole rows in one wave: H128 and sv here
        const uint16_t *svp = (const uint16_t *)(colgroup + 2048 * K + 256);  // record (nb, 0)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            float t[4][16];
#pragma unroll
            for (int cb = 0; cb < 4; ++cb)
#pragma unroll
                for (int e = 0; e < 16; ++e) t[cb][e] = acc[rb][cb][e];
            gemm_rows_out<16>(t, lane, mt * BM + 32 * RB * rw + 32 * rb, svp, rows, y, y_f16, y_stride,
                              (size_t)nb * 128, res, res_stride);
        }
    }
}

// Split-K reduction (split count > 1).  One workgroup of 4 waves per unit
// (tile, row block blk = RB wave + rb, vp): the 16 rows 32 blk + 16 vp .. +15 of
// the tile x its 128 columns.  Wave c sums column block c (32 columns) over the
// splits in fp32 in split order (so the result does not depend on the order the
// GEMM's workgroups ran in): per split one 16-byte load per lane, the SB splits
// of a batch in flight together; the sums go through LDS as [row][column], and wave w then
// finishes rows 4 w .. 4 w + 3 (h128_wave over the 128 columns, sv, the optional
// residual), lane l writing columns l and l + 64.
template <int RB, int W, int SB>
__global__ __launch_bounds__(256) void gemm_reduce_kernel(const uint16_t *__restrict__ partials,
                                                          const int *__restrict__ exps, int splits, int nbs,
                                                          const uint8_t *__restrict__ records, int bits, int kbs,
                                                          void *y, int y_f16, size_t y_stride, int rows, int nunits,
                                                          const void *res, size_t res_stride) {
    constexpr int BM = 32 * RB * W;
    constexpr size_t kPerSplit = (size_t)W * RB * 4 * 2 * 64 * 8;  // halves
    __shared__ float sums[16][129];  // [row][column], padded against bank conflicts
    const int lane = threadIdx.x & 63, c = threadIdx.x >> 6;
    const int u = blockIdx.x;
    if (u >= nunits) return;  // whole workgroups
    const int vp = u & 1, blk = (u >> 1) % (W * RB), tile = (u >> 1) / (W * RB);
    const int mt = tile / nbs, nb = tile - mt * nbs;
    const uint16_t *src = partials + (size_t)tile * splits * kPerSplit + (size_t)blk * 8 * 512 + (c * 2 + vp) * 512 +
                          lane * 8;
    float t[8];
#pragma unroll 1
    for (int sp0 = 0; sp0 < splits; sp0 += SB) {
        u4 in[SB];
        int ex[SB];  // each split's block exponent (the GEMM stored the block scaled by 2^-ex)
#pragma unroll
        for (int q = 0; q < SB; ++q) {
            const int sp = sp0 + q < splits ? sp0 + q : splits - 1;
            ex[q] = exps[(((size_t)tile * splits + sp) * (W * RB) + blk) * 4 + c];
            // non-temporal loads for the partials of tiles up to 256 rows (each is
            // read once: k = 14336, n = 4096 rows 100..200 -0.7 to -1.6 us per call,
            // rows 16..64 -0.1 to -0.4 us, k = 2048, n = 6144 rows 256 -3.1 us); the
            // 512-row tiles' partials load faster as plain loads (non-temporal:
            // M=512 +3.5 us)
            const u4 *ps = (const u4 *)(src + (size_t)sp * kPerSplit);
            if constexpr (BM <= 256) in[q] = __builtin_nontemporal_load(ps);
            else in[q] = *ps;
        }
#pragma unroll
        for (int q = 0; q < SB; ++q)
            if (sp0 + q < splits) {
                // 2^ex is exact and so is the product of a half by it: one fused
                // rounding per add, the same sum as scaling first and then adding
                const float sc = __builtin_amdgcn_ldexpf(1.0f, ex[q]);
                const uint32_t w[4] = {in[q].x, in[q].y, in[q].z, in[q].w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float h = half_bits_to_float((uint16_t)(w[e >> 1] >> (16 * (e & 1))));
                    t[e] = sp0 + q == 0 ? h * sc : __builtin_fmaf(h, sc, t[e]);
                }
            }
    }
    // element 8 vp + e of the 32x32 MFMA D block of lane l: row (e % 4) + 8 (e / 4) +
    // 4 (l / 32) of the unit's 16, column 32 c + l % 32
#pragma unroll
    for (int e = 0; e < 8; ++e) sums[(e & 3) + 8 * (e >> 2) + 4 * (lane >> 5)][32 * c + (lane & 31)] = t[e];
    __syncthreads();
    const uint16_t *svp = (const uint16_t *)(records + (size_t)nb * kbs * group_bytes(bits) + 2048 * bits + 256);
    const float sv0 = half_bits_to_float(svp[lane]), sv1 = half_bits_to_float(svp[lane + 64]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int rl = 4 * c + i, row = mt * BM + 32 * blk + 16 * vp + rl;
        float a0 = sums[rl][lane], a1 = sums[rl][lane + 64];
        h128_wave(a0, a1, lane);
        a0 *= sv0;
        a1 *= sv1;
        if (row < rows) {
            const size_t o = (size_t)row * y_stride + (size_t)nb * 128;
            if (res) {  // y = res + layer, one rounding
                const size_t ro = (size_t)row * res_stride + (size_t)nb * 128;
                if (y_f16) {
                    a0 += half_bits_to_float(((const uint16_t *)res)[ro + lane]);
                    a1 += half_bits_to_float(((const uint16_t *)res)[ro + lane + 64]);
                } else {
                    a0 += ((const float *)res)[ro + lane];
                    a1 += ((const float *)res)[ro + lane + 64];
                }
            }
            // non-temporal: k = 4096, n = 14336 M=512 -0.6 us, k = 2048, n = 6144 rows 256
            // -0.3 us, the rest within +-0.1 us
            if (y_f16) {
                __builtin_nontemporal_store(float_to_half_bits(a0), (uint16_t *)y + o + lane);
                __builtin_nontemporal_store(float_to_half_bits(a1), (uint16_t *)y + o + lane + 64);
            } else {
                __builtin_nontemporal_store(a0, (float *)y + o + lane);
                __builtin_nontemporal_store(a1, (float *)y + o + lane + 64);
            }
        }
    }
}

// Tile heights: 32 rows (4 waves: 4 column quarters), 64 rows (8 waves: 2 row
// waves x 4 column quarters), 128 (8 waves: 4 x 2 column halves with a k split,
// else 4 waves of one 32-row block each), 256 (4 waves, two blocks), 512 (8
// waves, two blocks): above 256 rows one 512-row tile decodes each record once
// for all rows where two 256-row tiles decode it twice.  The short tiles cut
// the padded MFMA work and activation loads of a 128-row one (rows 33..64 at
// k = 14336, n = 4096: 33.5 -> 27.7 us per call; rows 17..32 on 32-row tiles
// 22.7 us against 24.5 on 64-row ones); two 64-row tiles for rows 65..128
// decode every record twice and are slower (42 against 34 us).
int gemm_tile_rows(size_t rows) {
    return rows <= 32 ? 32 : rows <= 64 ? 64 : rows <= 128 ? 128 : rows <= 256 ? 256 : 512;
}

// k splits of a tile class: split k only below kGemmSplitTiles tiles (the split
// partials are summed by gemm_reduce_kernel), at most one split per record.
// 32- and 64-row tiles fill the CUs once (one workgroup each); 32-row tiles (4
// waves, 64 KB of LDS) run two per CU when each split keeps >= 4 records (rows
// 17..32 at k = 14336, n = 4096: 22.7 -> 21.2 us; at k <= 6144 two per CU with
// 1..2 records each were 1.5-3 us slower than one).  For 128..512-row tiles
// the count minimises records per split x the tile's measured time per record
// (1.15 / 1.73 / 2.83 us) + split-partial bytes at 0.6 us per MB (written by
// the GEMM, read by the reduction), within one workgroup per CU.  Measured
// sweeps over splits 1..32 (k = 2048 / 6144 / 14336, n = 512..6144, rows
// 24..512) put this rule within 1 us of each shape's best count; against at
// least 4 records per split it takes k = 2048, n = 512 at rows 300 from 23.4
// to 18.8 us and k = 2048, n = 2048 at rows 24 from 13.7 to 11.6 us.
static int gemm_splits(int kbs, int tiles, int bm) {
    if (tiles >= (int)kGemmSplitTiles) return 1;
    int s;
    if (bm <= 64) {
        int wgs = kGemmTargetWgs;
        if (bm == 32 && kbs / ((2 * kGemmTargetWgs + tiles - 1) / tiles) >= 4) wgs = 2 * kGemmTargetWgs;
        s = 2 * tiles > wgs ? (wgs + tiles - 1) / tiles : wgs / tiles;
        if (s < kbs) {  // the fewest splits with the same records per split
            const int per = (kbs + s - 1) / s;
            s = (kbs + per - 1) / per;
        }
    } else {
        const double per_record_us = bm == 128 ? 1.15 : bm == 256 ? 1.73 : 2.83;
        const int smax = kGemmTargetWgs / tiles > 1 ? kGemmTargetWgs / tiles : 1;
        double best = 0.0;
        s = 1;
        for (int c = 1; c <= smax && c <= kbs; ++c) {
            const double partial_mb = c > 1 ? (double)tiles * c * bm * 256 * 1e-6 : 0.0;
            const double t = per_record_us * ((kbs + c - 1) / c) + 0.6 * partial_mb;
            if (c == 1 || t < best) best = t, s = c;
        }
    }
    return s < 1 ? 1 : (s > kbs ? kbs : s);
}

static GemmPlan gemm_plan_bm(size_t k, size_t n, size_t rows, int bm) {
    GemmPlan p{};
    p.nbs = (int)(n / 128);
    p.kbs = (int)(k / 128);
    p.bm = bm;
    p.mtiles = (int)((rows + p.bm - 1) / p.bm);
    const int tiles = p.nbs * p.mtiles;
    const int s = gemm_splits(p.kbs, tiles, p.bm);
    if (p.bm < 128 && s == 1) return gemm_plan_bm(k, n, rows, 128);  // the 32/64-row tiles need a split
    p.splits = s;
    size_t off = kSharedPrefixBytes;  // the GEMM leaves the GEMV exchange alone
    p.xh_off = off;
    off += ((size_t)p.mtiles * p.bm * k * 2 + 255) & ~(size_t)255;
    p.partials_off = off;
    if (s > 1) off += (size_t)tiles * s * p.bm * 128 * 2;  // fp16 partials
    p.exps_off = off;
    if (s > 1) off += ((size_t)tiles * s * (p.bm / 32) * 4 * 4 + 255) & ~(size_t)255;  // one per 32x32 block
    p.bytes = (off + 255) & ~(size_t)255;
    return p;
}

GemmPlan gemm_plan(size_t k, size_t n, size_t rows) { return gemm_plan_bm(k, n, rows, gemm_tile_rows(rows)); }

// one tile class: kernel <RB, W> (NSG scheduling groups per k-step, XD activation
// k-steps in flight) and its reduction
template <int K, int CB, int RB, int W, int NSG, int XD, int CH>
static void launch_gemm_tiles(const uint8_t *rec, size_t k, uint16_t *xh, size_t rows, void *y, int y_f16,
                              size_t y_stride, uint8_t *ws, const GemmPlan &p, hipStream_t stream, const void *res,
                              size_t res_stride) {
    constexpr int WR = W / CH;  // the reduction sees the row waves
    static_assert(32 * RB * WR == 32 || 32 * RB * WR == 64 || 32 * RB * WR == 128 || 32 * RB * WR == 256 || 32 * RB * WR == 512,
                  "tile height");
    const dim3 grid((unsigned)(p.mtiles * p.nbs * p.splits)), block(W * 64);
    uint16_t *part = (uint16_t *)(ws + p.partials_off);
    int *exps = (int *)(ws + p.exps_off);
    const int nunits = p.mtiles * p.nbs * (p.bm / 16);  // reduction: one 4-wave workgroup per 16 rows of a tile
    const int kq = p.kbs / p.splits, kr = p.kbs % p.splits;
    gemm_kernel<K, CB, RB, W, NSG, XD, CH><<<grid, block, 0, stream>>>(
        rec, p.kbs, p.nbs, p.mtiles, p.splits, kq, kr, xh, k, part, exps, y, y_f16, y_stride, (int)rows, res,
        res_stride);
    if (p.splits > 1)
    {  // SB splits' loads in flight per batch: one batch for up to 16 splits (the
       // 32-row tiles' 16: -0.4 to -0.6 us per call against two batches of 8)
        if (p.splits > 8)
            gemm_reduce_kernel<RB, WR, 16><<<dim3((unsigned)nunits), dim3(256), 0, stream>>>(
                part, exps, p.splits, p.nbs, rec, K, p.kbs, y, y_f16, y_stride, (int)rows, nunits, res, res_stride);
        else
            gemm_reduce_kernel<RB, WR, 8><<<dim3((unsigned)nunits), dim3(256), 0, stream>>>(
                part, exps, p.splits, p.nbs, rec, K, p.kbs, y, y_f16, y_stride, (int)rows, nunits, res, res_stride);
    }
}

template <int K, int CB>
static void launch_gemm_kc(const uint8_t *rec, size_t k, uint16_t *xh, size_t rows, void *y, int y_f16,
                           size_t y_stride, uint8_t *ws, const GemmPlan &p, hipStream_t stream, const void *res,
                           size_t res_stride) {
    if (p.bm == 32)  // 4 waves: 4 column quarters (the plan gives it a split)
        launch_gemm_tiles<K, CB, 1, 4, 0, 8, 4>(rec, k, xh, rows, y, y_f16, y_stride, ws, p, stream, res, res_stride);
    else if (p.bm == 64)  // 8 waves: 2 row waves x 4 column quarters (the plan gives it a split)
        launch_gemm_tiles<K, CB, 1, 8, 0, 8, 4>(rec, k, xh, rows, y, y_f16, y_stride, ws, p, stream, res, res_stride);
    else if (p.bm == 128 && p.splits > 1)  // 8 waves: 4 row waves x 2 column halves, two waves per SIMD
        launch_gemm_tiles<K, CB, 1, 8, 0, 8, 2>(rec, k, xh, rows, y, y_f16, y_stride, ws, p, stream, res, res_stride);
    else if (p.bm == 128)
        launch_gemm_tiles<K, CB, 1, 4, 8, 8, 1>(rec, k, xh, rows, y, y_f16, y_stride, ws, p, stream, res, res_stride);
    else if (p.bm == 256)
        launch_gemm_tiles<K, CB, 2, 4, 8, 8, 1>(rec, k, xh, rows, y, y_f16, y_stride, ws, p, stream, res, res_stride);
    else  // 8 waves: no scheduling groups, four activation k-steps in flight (measured best at M = 512)
        launch_gemm_tiles<K, CB, 2, 8, 0, 4, 1>(rec, k, xh, rows, y, y_f16, y_stride, ws, p, stream, res, res_stride);
}

template <int K>
static hipError_t launch_gemm_k(const void *records, int cb, size_t k, const void *x, int x_f16, size_t rows,
                                size_t x_stride, void *y, int y_f16, size_t y_stride, uint8_t *ws, const GemmPlan &p,
                                hipStream_t stream, const void *res, size_t res_stride) {
    const uint8_t *rec = (const uint8_t *)records;
    uint16_t *xh = (uint16_t *)(ws + p.xh_off);
    const int rows_padded = p.mtiles * p.bm;
    gemm_xprep_kernel<<<dim3(p.kbs, rows_padded / 8), dim3(64), 0, stream>>>(rec, K, x, x_f16, x_stride, (int)rows,
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
