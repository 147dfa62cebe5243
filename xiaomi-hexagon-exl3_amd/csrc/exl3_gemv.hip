// exl3_gemv.hip -- the EXL3 layer at rows 1..32 on gfx950 (gemv_kernel,
// gemv_xprep_kernel): each lane decodes 32 trellis positions of a tile straight
// into fp16 MFMA A-fragments (W^T), v_mfma_f32_16x16x32_f16 accumulates in fp32;
// split-K partials are reduced in fixed order by the last split's workgroup of
// each 128-column group, which applies H128 and sv.
// Reference semantics: src/exl3-ggml.cpp:51-92.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include <atomic>
#include <type_traits>

#include "exl3_kernel_common.hpp"

namespace exl3k {

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
//      split-K partials are reduced in split order by the workgroup of the
//      column group's last split, which applies H128 and sv
//      (src/exl3-ggml.cpp:84-90).
template <int K>
struct GemvStream {
    static constexpr int DEPTH = K <= 2 ? 12 : (K <= 4 ? 8 : 4);  // groups in flight per wave
};
// Phase stamps, in the diagnostic library only (libexl3_hip_stamps.so, built with
// EXL3_PHASE_STAMPS): at each phase of the call thread 0 of the workgroup puts
// the 100 MHz s_memrealtime counter into a 64-byte LDS slot, and at its end
// copies the slot to g_exl3_gemv_stamps[workgroup][phase] (workgroup = x + nbs
// y in dispatch order) with ordinary vector stores: no global store sits
// between the phases for a later wait on memory to include, and no register
// stays live across the kernel for the stamps.  Every call overwrites what its
// workgroups reach; after a stream of equal calls the array holds the last
// one.  Phases: 0 start, 1 prep barrier passed, 2 every wave's main loop done,
// 3 partial ready (a writer: its words issued; the summing workgroup: its own
// partial in LDS), 4 the other splits' words of row 0 read, 5 row 0's output
// issued, 6 the exchange cleared (4..6: summing workgroups only).
#ifdef EXL3_PHASE_STAMPS
constexpr int kStampPhases = 8;
constexpr unsigned kStampWorkgroups = 8192;
__device__ uint64_t g_exl3_gemv_stamps[kStampWorkgroups * kStampPhases];
struct PhaseStamps {
    uint64_t *slot;
    __device__ __forceinline__ void mark(int phase) {
        if (threadIdx.x == 0) slot[phase] = __builtin_amdgcn_s_memrealtime();
    }
    __device__ __forceinline__ void flush(int phases) {
        const unsigned w = blockIdx.x + gridDim.x * blockIdx.y;
        if (threadIdx.x == 0 && w < kStampWorkgroups)
            for (int p = 0; p < phases; ++p) g_exl3_gemv_stamps[w * kStampPhases + p] = slot[p];
    }
};
#define EXL3_STAMPS_DECLARE                                    \
    __shared__ uint64_t stamp_slot[kStampPhases];              \
    PhaseStamps stamps{stamp_slot};
#else
struct PhaseStamps {
    __device__ __forceinline__ void mark(int) {}
    __device__ __forceinline__ void flush(int) {}
};
#define EXL3_STAMPS_DECLARE PhaseStamps stamps;
#endif

constexpr int kGemvPrepMax = 16;          // a workgroup preps at most kGemvPrepMax x waves (kb, row) blocks
constexpr size_t kGemvDummyBytes = 8192;  // >= largest lane offset of a group + its K words (1024 K)
constexpr size_t kGemvFragLds = 49152;    // LDS budget of the B fragments of a workgroup (rows <= 8)
constexpr size_t kGemvFragLds16 = 65536;  // the same for rows 9..16 (two workgroups still fit a CU)

// MODE 0 (rows 1..8): one block of 16 B columns, hi and lo of 8 rows.
// MODE 1 (rows 9..16): a second block of B columns carries rows 8..15 (hi and lo as
// for rows 0..7); each decoded A fragment feeds both blocks' MFMAs, so the decode
// is shared by all 16 rows.
// MODE 2 (rows 17..32): two blocks of 16 rows each, fp16 activations without the
// lo halves, prepared once per call by gemv_xprep_kernel (xpre) and copied into
// LDS instead of being transformed again by every column group.
// amdgpu_waves_per_eu(4): two workgroups per CU.  Without it the compiler places
// the VGPR that holds spilled SGPRs (rows 17..32) at v222, and the kernel then
// runs one workgroup per CU.
template <int K, int CB, int MODE>
__global__ __launch_bounds__(kGemvWaves * 64) __attribute__((amdgpu_waves_per_eu(4))) void gemv_kernel(
    GemvTargets tg, int kbs, int splits, int kq, int kr, const void *__restrict__ x, int x_f16, size_t x_stride,
    int rows, const uint8_t *__restrict__ dummy, uint32_t *__restrict__ partials, int y_f16,
    const uint8_t *__restrict__ xpre, uint32_t *__restrict__ status, int spin_limit, int drop_split) {
    constexpr bool TWO = MODE >= 1, HILO = MODE <= 1;
    constexpr int W = kGemvWaves;
    constexpr int P = W / 4;  // waves per column pair
    constexpr int NT = W * 64;
    constexpr size_t GB = (size_t)2048 * K + 512;
    // rows 9..16 need 8 more accumulator and fragment registers: a shorter ring at
    // K <= 2 keeps them within 128 VGPRs (two workgroups per CU)
    constexpr int D = TWO && K <= 2 ? 8 : GemvStream<K>::DEPTH;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint8_t *frag = smem;
    // B fragments of one (kb, r4, half): [kg][hl][row] x 16 bytes (MODE 2: [kg][row])
    const int blk_bytes = (HILO ? 128 : 64) * rows;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int cp = wave & 3, part = wave >> 2;
    // grid (column group, split): no division on the way to the first loads.
    // Split s owns kq + (s < kr) records from kb0 (kq = kbs / splits, kr = kbs % splits)
    const int nb = blockIdx.x, s = blockIdx.y;
    EXL3_STAMPS_DECLARE
    stamps.mark(0);
    // The 9..16-row prep (hi and lo fragments of up to 16 rows) is long enough
    // that, at equal priority, a CU's second workgroup runs it mostly in the
    // issue gaps of the first one's decode (the older waves issue first): raised
    // until the prep barrier it no longer trails by microseconds (rows 12 and 16
    // -1.3 to -1.9 us per call; no gain at 8 rows or fewer, a loss at 17..32)
    if constexpr (MODE == 1) __builtin_amdgcn_s_setprio(1);
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
        // the first weight-ring slot right behind the activation loads: its
        // latency then passes under this prep's H128 work (the one-block prep
        // below is too short for that and issues it after the barrier)
        load_chunk<K>(group_src(0), buf[0]);
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
                // cross-lane stages in signed form: the butterfly sgn v + v' is
                // sgn (v + sgn v'), so each stage keeps m = m + sgn dpp(m) and the
                // stage signs multiply into one lane sign, applied with the
                // 1/sqrt(128) scale; the same roundings as sgn v + v'.  With two or
                // more units per wave each value is one DPP fmac (dpp_block_stage8:
                // rows 8 -0.75 us, rows 14 -0.5 us per call at k = 14336); one unit
                // keeps the compiler's DPP move + fma (the fused blocks were 0.3 us
                // slower at rows 2)
                if constexpr (NQ >= 2) {
                    dpp_block_stage8<1>(v, (pi & 1) ? -1.f : 1.f);
                    dpp_block_stage8<2>(v, (pi & 2) ? -1.f : 1.f);
                    dpp_block_stage8<4>(v, (pi & 4) ? -1.f : 1.f);
                    dpp_block_stage8<8>(v, (pi & 8) ? -1.f : 1.f);
                } else {
                    auto lane_stage = [&](auto sc) {
                        constexpr int S = decltype(sc)::value;
                        const float sgn = (pi & S) ? -1.f : 1.f;
#pragma unroll
                        for (int j = 0; j < 8; ++j) v[j] = __builtin_fmaf(dpp_block_xor<S>(v[j]), sgn, v[j]);
                    };
                    lane_stage(std::integral_constant<int, 1>{});
                    lane_stage(std::integral_constant<int, 2>{});
                    lane_stage(std::integral_constant<int, 4>{});
                    lane_stage(std::integral_constant<int, 8>{});
                }
                const float scale = (__builtin_popcount(pi & 15) & 1) ? -0.08838834764831844055f
                                                                       : 0.08838834764831844055f;
                const int blk = (4 * q + g) * W + wave;
                if (blk < nblk) {
                    const int kbl = blk / rows, r = blk - kbl * rows;
                    h8 hi, lo;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        // opaque product: hi and lo must both come from this binary32
                        // value (the compiler otherwise rounds x * scale straight to
                        // fp16 in a v_fma_mix for the lo term and stores hi rounded from
                        // binary32, which can disagree by one fp16 ulp)
                        const float e = mul_rn_f32(v[j], scale);
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
            asm("" : "+v"(a), "+v"(b));  // hi and lo from these binary32 values (as above)
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
    stamps.mark(1);
    if constexpr (MODE == 1) __builtin_amdgcn_s_setprio(0);
    if (MODE == 2 || nblk <= W) load_chunk<K>(group_src(0), buf[0]);  // not issued by the prep
#pragma unroll
    for (int d = 1; d < D; ++d) load_chunk<K>(group_src(d), buf[d]);

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
    stamps.mark(2);
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
    // the workgroup's partial: element t = row * 128 + column, the P wave partials summed
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
    float *own = red + P * nval;  // the workgroup partial, for the output rows
    if (splits > 1) {
        uint32_t *all = partials + (size_t)nb * splits * (size_t)nval;
        if (s != splits - 1) {  // hand the partial over and end
            if (s == drop_split) return;  // failure injection (tests only): this partial never arrives
            uint32_t *mine = all + (size_t)s * nval;
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int t = tid + i * NT;
                if (t < nval) store_exchange(mine + t, psum[i]);
            }
            stamps.mark(3);
            stamps.flush(4);
            return;
        }
        // the last split: wave r sums row r's elements lane and lane + 64 over
        // the splits in split order, its own partial (from LDS) last, a batch of
        // splits' loads in flight together, straight into the registers of the
        // output transform.  A word still empty is read again (with the rest of
        // its batch) until it is full, or until the wave's budget of polls runs
        // out or another wave of the workgroup has given up (`gave_up`).  A
        // workspace whose status word is set gives NaN without waiting.
        int *gave_up = (int *)(own + nval);  // LDS, after the workgroup partial
        const uint32_t poisoned = load_exchange(status);
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int t = tid + i * NT;
            if (t < nval) own[t] = psum[i];
        }
        if (tid == 0) *gave_up = poisoned != 0u;
        __syncthreads();
        stamps.mark(3);
        const int nsp = splits - 1;  // splits in the exchange
        int budget = spin_limit;
        for (int rr = wave; rr < rows; rr += W) {
            constexpr int B = 16;
            float a0 = 0.f, a1 = 0.f;
            for (int base = 0; base < nsp; base += B) {
                uint32_t v0[B], v1[B];
                auto load_batch = [&](int bs, int rw) {
#pragma unroll
                    for (int jb = 0; jb < B; ++jb) {
                        const int sp = bs + jb < nsp ? bs + jb : nsp - 1;  // repeats are not used
                        const uint32_t *q = all + (size_t)sp * nval + rw * 128 + lane;
                        v0[jb] = load_exchange(q);
                        v1[jb] = load_exchange(q + 64);
                    }
                };
                load_batch(base, rr);
                auto any_empty = [&]() {
                    int z = 0;
#pragma unroll
                    for (int jb = 0; jb < B; ++jb)
                        if (base + jb < nsp) z |= (v0[jb] == 0u) | (v1[jb] == 0u);
                    return z != 0;
                };
                while (__builtin_amdgcn_ballot_w64(any_empty())) {
                    if (__hip_atomic_load(gave_up, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) break;
                    if (--budget < 0) {
                        __hip_atomic_store(gave_up, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(2);
                    // the addresses are formed again in every pass (the empty asm hides
                    // that they repeat), so they hold no registers across the loop
                    int bs = base, rw = rr;
                    asm volatile("" : "+s"(bs), "+s"(rw));
                    load_batch(bs, rw);  // a full word keeps its value until the clearing below
                }
#pragma unroll
                for (int jb = 0; jb < B; ++jb)
                    if (base + jb < nsp) {  // a word that never filled: a loud result, not a hang
                        a0 += v0[jb] && !poisoned ? exchange_value(v0[jb]) : __builtin_nanf("");
                        a1 += v1[jb] && !poisoned ? exchange_value(v1[jb]) : __builtin_nanf("");
                    }
            }
            if (rr == 0) stamps.mark(4);
            finish_row(rr, a0 + own[rr * 128 + lane], a1 + own[rr * 128 + lane + 64]);
            if (rr == 0) stamps.mark(5);
        }
        // every word has been read: empty them for the next call; after a give-up
        // a partial may still arrive, so the status word marks the workspace
        __syncthreads();
        if (tid == 0 && *gave_up && !poisoned) __hip_atomic_store(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // nval is a multiple of 128 words and `all` 512-byte aligned: whole 16-byte units
        for (int t = 4 * tid; t < nsp * nval; t += 4 * NT) clear_exchange4(all + t);
        stamps.mark(6);
        stamps.flush(7);
        return;
    }
    // 6. (one workgroup per column group) output H128 per row from the LDS sums
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int t = tid + i * NT;
        if (t < nval) own[t] = psum[i];
    }
    __syncthreads();
    stamps.mark(3);
    for (int rr = wave; rr < rows; rr += W) finish_row(rr, own[rr * 128 + lane], own[rr * 128 + lane + 64]);
    stamps.flush(4);
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
// the P partials, the output rows and the summing workgroup's give-up flag
static size_t gemv_lds_bytes(int nkb_max, size_t rows) {
    const size_t frag = (size_t)nkb_max * gemv_frag_bytes_per_kb(rows);
    const size_t red = (size_t)(kGemvWaves / 4 + 1) * rows * 128 * 4 + 16;
    return ((frag > red ? frag : red) + 15) & ~(size_t)15;
}

GemvPlan gemv_plan(size_t k, size_t n, size_t rows) {
    GemvPlan p{};
    p.nbs = (int)(n / 128);
    p.kbs = (int)(k / 128);
    // about four records per workgroup (a workgroup's fixed latency chain then
    // stays small against its stream), between 256 and 512 workgroups (one to two
    // per CU), and the fewest splits with the same records per split.  Measured
    // best or within 0.1 us of the best split count at rows 1 and 8 for k = 2048
    // (n = 512, 2048, 6144; q/k/v 2048 + 512 + 512 and gate/up 2 x 6144 grouped),
    // 6144 x 2048, 4096 x 14336 and 14336 x 4096; against a floor of 128
    // workgroups, k = 6144, n = 2048 -0.3 us and the q/k/v group at rows 8 -0.7 us
    int s = (p.kbs + 3) / 4;
    if (p.nbs * s > 512) s = 512 / p.nbs;
    if (p.nbs * s < 256) s = 256 / p.nbs;
    s = s < 1 ? 1 : (s > p.kbs ? p.kbs : s);
    s = (p.kbs + (p.kbs + s - 1) / s - 1) / ((p.kbs + s - 1) / s);
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
    p.partials_off = 0;  // the exchange
    p.exchange_bytes = s > 1 ? (size_t)p.nbs * s * rows * 128 * 4 : 0;  // one 32-bit word per partial value
    p.fits = p.exchange_bytes <= kGemvExchangeBytes;
    size_t off = kSharedPrefixBytes;
    p.dummy_off = off;  // target of the stream's issues past a wave's last group (loaded, never used)
    off += kGemvDummyBytes;
    p.xpre_off = off;  // rows > 16: prepared activations of up to kGemvMaxTargets matrices
    if (rows > 16) off += (size_t)kGemvMaxTargets * p.kbs * gemv_frag_bytes_per_kb(rows);
    p.bytes = (off + 255) & ~(size_t)255;
    return p;
}

bool gemv_serves(size_t k, size_t n, size_t rows) {
    return rows >= 1 && rows <= (size_t)kGemvMaxRows && gemv_plan(k, n, rows).fits;
}

bool gemv_serves_single(size_t k, size_t n, size_t rows) {
    if (!gemv_serves(k, n, rows)) return false;
    if (rows <= (size_t)kGemvSingleMaxRows) return true;
    // rows 15..16 (the two-block hi/lo GEMV) when a workgroup's prep is short
    return rows <= 16 && (size_t)gemv_plan(k, n, rows).nkw * rows <= (size_t)kGemvSinglePrepBlocks;
}

static std::atomic<int> g_fault_spin_limit{0}, g_fault_drop_split{-1};

void set_exchange_fault(int spin_limit, int drop_split) {
    g_fault_spin_limit.store(spin_limit > 0 ? spin_limit : 0, std::memory_order_relaxed);
    g_fault_drop_split.store(drop_split >= 0 ? drop_split : -1, std::memory_order_relaxed);
}
int exchange_spin_limit() {
    const int spin = g_fault_spin_limit.load(std::memory_order_relaxed);
    return spin > 0 ? spin : kExchangeSpinLimit;
}
int exchange_drop_split() { return g_fault_drop_split.load(std::memory_order_relaxed); }

template <int K, int CB>
static hipError_t launch_gemv_kc(const GemvTargets &tg, const void *x, int x_f16, size_t rows, size_t x_stride,
                                 int y_f16, uint8_t *ws, const GemvPlan &p, hipStream_t stream) {
    const size_t lds = gemv_lds_bytes(p.nkw, rows);
    // x fastest: workgroup (nb, s) is dispatched as nb + s nbs, as a 1-D grid would
    // be, so the last split's workgroups, which wait for the others, come last
    const dim3 grid((unsigned)p.nbs, (unsigned)p.splits), block(kGemvWaves * 64);
    const int kq = p.kbs / p.splits, kr = p.kbs % p.splits;
    uint32_t *part = (uint32_t *)(ws + p.partials_off);
    uint32_t *status = (uint32_t *)(ws + kStatusOffset);
    const int spin_limit = exchange_spin_limit();
    const int drop_split = exchange_drop_split();
    if (rows > 16) {
        uint16_t *xp = (uint16_t *)(ws + p.xpre_off);
        gemv_xprep_kernel<<<dim3((unsigned)((rows + 3) / 4), (unsigned)p.kbs, (unsigned)tg.count), dim3(256), 0,
                            stream>>>(tg, K, x, x_f16, x_stride, (int)rows, p.kbs, xp);
        gemv_kernel<K, CB, 2><<<grid, block, lds, stream>>>(tg, p.kbs, p.splits, kq, kr, x, x_f16, x_stride,
                                                            (int)rows, ws + p.dummy_off, part, y_f16,
                                                            (const uint8_t *)xp, status, spin_limit, drop_split);
    } else if (rows > 8) {
        gemv_kernel<K, CB, 1><<<grid, block, lds, stream>>>(tg, p.kbs, p.splits, kq, kr, x, x_f16, x_stride,
                                                            (int)rows, ws + p.dummy_off, part, y_f16, nullptr,
                                                            status, spin_limit, drop_split);
    } else {
        gemv_kernel<K, CB, 0><<<grid, block, lds, stream>>>(tg, p.kbs, p.splits, kq, kr, x, x_f16, x_stride,
                                                            (int)rows, ws + p.dummy_off, part, y_f16, nullptr,
                                                            status, spin_limit, drop_split);
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

}  // namespace exl3k

#ifdef EXL3_PHASE_STAMPS
// The diagnostic library's one extra export: copies up to `count` stamps
// ([workgroup][8 phases], 100 MHz ticks) of the current device into `out`.
extern "C" __attribute__((visibility("default"))) int exl3_hip_debug_gemv_stamps(uint64_t *out, size_t count) {
    const size_t all = (size_t)exl3k::kStampWorkgroups * exl3k::kStampPhases;
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(exl3k::g_exl3_gemv_stamps), (count < all ? count : all) * 8) ==
                   hipSuccess
               ? 0
               : -1;
}
#endif
