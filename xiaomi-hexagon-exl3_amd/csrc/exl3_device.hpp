// exl3_device.hpp -- gfx950 device primitives for EXL3 trellis decode.
//
// Bitstream facts (src/exl3_codec.cpp:88-113, restated):
//   * a 16x16 tile is 16*K little-endian u16 = 8*K u32 words; word i is
//     u16[2i] | u16[2i+1] << 16 and stream bit b is bit 31 - (b % 32) of word b / 32;
//   * the stream is cyclic (256*K bits); position p (0..255) has the state formed
//     by the 16 stream bits ending (exclusive) at bit (p + 1) * K;
//   * position p = 8 L + e sits at row 2 (L % 4) + (e & 1) + 8 ((e >> 1) & 1),
//     column L / 4 + 8 ((e >> 2) & 1) of the tile.
//
// A "run" is the 16 consecutive positions p0 = 32 c + 16 h .. p0 + 15 (c in 0..7,
// h in 0..1).  It covers tile columns c and c + 8 at the 8 rows
//   h = 0: {0, 1, 8, 9, 2, 3, 10, 11}      h = 1: {4, 5, 12, 13, 6, 7, 14, 15}
// (run index i -> e = i % 8, q = 2h + i / 8).  One lane decodes one run from the
// 3..6 stream words that hold it, entirely in registers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace exl3dev {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

template <typename T, typename F>
__device__ __forceinline__ T bitcast(F v) { return __builtin_bit_cast(T, v); }

// ---------------------------------------------------------------- codebooks
// src/exl3_codec.cpp:68-86.  mul1: s = byte sum of state * 0x83dcd12d,
// w = fp16(fma(fp16(1024 + s), fp16 0x1eee, fp16 0xc931)); that fma is exact in
// binary32, so one fp16 fma (exact product-sum, one RNE) gives the same bits.
// mcg / 3inst: P' = (P & 0x8fff8fff) ^ 0x3b603b60, w = fp16(P'.lo) + fp16(P'.hi)
// (exact sum, one RNE).
template <int CB>
__device__ __forceinline__ uint32_t trellis_hash(uint32_t s) {
    if constexpr (CB == 2) return s * 0x83dcd12du;
    else if constexpr (CB == 1) return s * 0xcbac1fedu;
    else return s * 89226354u + 64248484u;
}

// two 16-bit states (upper bits of the arguments are ignored) -> packed fp16
// pair, first state in the low half
template <int CB>
__device__ __forceinline__ uint32_t codebook_pair(uint32_t sa, uint32_t sb) {
    const uint32_t pa = trellis_hash<CB>(sa & 0xffffu), pb = trellis_hash<CB>(sb & 0xffffu);
    if constexpr (CB == 2) {
        const uint32_t hsum = __builtin_amdgcn_sad_hi_u8(pb, 0u, __builtin_amdgcn_sad_u8(pa, 0u, 0x64006400u));
        const h2 w = __builtin_elementwise_fma(bitcast<h2>(hsum), bitcast<h2>(0x1eee1eeeu), bitcast<h2>(0xc931c931u));
        return bitcast<uint32_t>(w);
    } else {
        const uint32_t qa = (pa & 0x8fff8fffu) ^ 0x3b603b60u, qb = (pb & 0x8fff8fffu) ^ 0x3b603b60u;
        const uint32_t lo = __builtin_amdgcn_perm(qb, qa, 0x05040100u);  // [qb.lo : qa.lo]
        const uint32_t hi = __builtin_amdgcn_perm(qb, qa, 0x07060302u);  // [qb.hi : qa.hi]
        return bitcast<uint32_t>(bitcast<h2>(lo) + bitcast<h2>(hi));
    }
}

template <int CB>
__device__ __forceinline__ uint16_t codebook_one(uint32_t s) {
    return (uint16_t)(codebook_pair<CB>(s, s) & 0xffffu);
}

// ------------------------------------------------------------- run geometry
// Window of a run after normalisation: it starts at bit OFF of word w[0] and
// spans NW words.  For even K every lane's run starts K + 16 bits into the word
// before word c*K (h = 0) or at the same offset of a later word (h = 1).  For odd
// K the h = 1 runs start 16 bits earlier in their word; those lanes load one more
// word and funnel-shift by 16 so all lanes share OFF.
template <int K>
struct RunGeo {
    static constexpr int OFF = K + 16;
    static constexpr int NW = (OFF + 15 * K + 16 + 31) / 32;
    static constexpr int WORDS = 8 * K;          // u32 words per tile
    static constexpr bool ODD = (K & 1) != 0;
    static constexpr int NLOAD = ODD ? NW + 1 : NW;
    // first loaded word (relative to c*K) for h = 0 and h = 1
    static constexpr int BASE0 = ODD ? -2 : -1;
    static constexpr int BASE1 = ODD ? (17 * K - 16) / 32 - 1 : (17 * K - 16) / 32;
};

// Byte offsets, within a tile, of the NLOAD words a run (c, h) reads.  They
// depend only on the lane, so kernels compute them once.  Indices wrap at both
// ends: the stream is cyclic (run c = 0, h = 0 reads the last word; for odd K
// the extra normalisation word of run c = 7, h = 1 is word 0).
template <int K>
__device__ __forceinline__ void run_word_offsets(int c, int h, uint32_t (&off)[RunGeo<K>::NLOAD]) {
    using G = RunGeo<K>;
    const int base = c * K + (h ? G::BASE1 : G::BASE0);
#pragma unroll
    for (int j = 0; j < G::NLOAD; ++j) {
        int idx = base + j;
        idx = idx < 0 ? idx + G::WORDS : idx;
        idx = idx >= G::WORDS ? idx - G::WORDS : idx;
        off[j] = (uint32_t)idx * 4u;
    }
}

// Load a run's words (tile = first byte of the tile, off from run_word_offsets
// plus any lane-constant byte offset) and normalise them so that the window
// starts at bit OFF of w[0] on every lane.
template <int K>
__device__ __forceinline__ void load_run(const uint8_t *__restrict__ tile, const uint32_t (&off)[RunGeo<K>::NLOAD],
                                         int h, uint32_t (&w)[RunGeo<K>::NW]) {
    using G = RunGeo<K>;
    uint32_t v[G::NLOAD];
#pragma unroll
    for (int j = 0; j < G::NLOAD; ++j) v[j] = __builtin_nontemporal_load((const uint32_t *)(tile + off[j]));
    if constexpr (G::ODD) {
        const uint32_t sh = h ? 16u : 0u;  // alignbit(a, b, 0) == b
#pragma unroll
        for (int j = 0; j < G::NW; ++j) w[j] = __builtin_amdgcn_alignbit(v[j], v[j + 1], sh);
    } else {
#pragma unroll
        for (int j = 0; j < G::NW; ++j) w[j] = v[j];
    }
}

template <int K>
__device__ __forceinline__ void load_run_words(const uint32_t *__restrict__ tile, int c, int h,
                                               uint32_t (&w)[RunGeo<K>::NW]) {
    uint32_t off[RunGeo<K>::NLOAD];
    run_word_offsets<K>(c, h, off);
    load_run<K>((const uint8_t *)tile, off, h, w);
}

// State i (0..15) of a run: 16 bits ending at window bit OFF + 16 + i*K,
// returned in the low 16 bits (upper bits are junk).
template <int K, int I>
__device__ __forceinline__ uint32_t run_state(const uint32_t (&w)[RunGeo<K>::NW]) {
    constexpr int E = RunGeo<K>::OFF + 16 + I * K;
    constexpr int S = E - 16;
    constexpr int J = S / 32;
    if constexpr ((E - 1) / 32 == J) {
        return w[J] >> (32 * (J + 1) - E);
    } else {
        return __builtin_amdgcn_alignbit(w[J], w[J + 1], 32 * (J + 2) - E);
    }
}

// Decode one run into the two fp16 MFMA A-operand fragments:
//   a1 = column c  rows R_h(0..7) as 4 packed pairs (slot 2v in the low half)
//   a2 = column c+8 rows R_h(0..7)
// with R_0 = {0,1,8,9,2,3,10,11}, R_1 = {4,5,12,13,6,7,14,15}.
// Run index i -> (q' = i / 8, e = i % 8): a1 takes e < 4, slot 4 q' + e;
// a2 takes e >= 4, slot 4 q' + e - 4.
template <int K, int CB>
__device__ __forceinline__ void decode_run(const uint32_t (&w)[RunGeo<K>::NW], u4 &a1, u4 &a2) {
    a1.x = codebook_pair<CB>(run_state<K, 0>(w), run_state<K, 1>(w));
    a1.y = codebook_pair<CB>(run_state<K, 2>(w), run_state<K, 3>(w));
    a2.x = codebook_pair<CB>(run_state<K, 4>(w), run_state<K, 5>(w));
    a2.y = codebook_pair<CB>(run_state<K, 6>(w), run_state<K, 7>(w));
    a1.z = codebook_pair<CB>(run_state<K, 8>(w), run_state<K, 9>(w));
    a1.w = codebook_pair<CB>(run_state<K, 10>(w), run_state<K, 11>(w));
    a2.z = codebook_pair<CB>(run_state<K, 12>(w), run_state<K, 13>(w));
    a2.w = codebook_pair<CB>(run_state<K, 14>(w), run_state<K, 15>(w));
}

// Row of run slot j (0..7) in half h: 4h + 2 (j / 4) + (j & 1) + 8 ((j >> 1) & 1)
__device__ __forceinline__ int run_slot_row(int h, int j) {
    return 4 * h + 2 * (j >> 2) + (j & 1) + 8 * ((j >> 1) & 1);
}

// ----------------------------------------------------------------- H128
// 128-point natural-order Walsh-Hadamard butterflies over v[0..127] in LDS,
// cooperatively by nthreads threads of the block (tid < nthreads), then the
// 1/sqrt(128) scale; same stage order as src/exl3_codec.cpp:153-165.
// The caller must __syncthreads() before (data written) -- this function ends
// with a barrier.
__device__ __forceinline__ void h128_lds(float *v, int rows, int stride, int tid, int nthreads) {
    for (int step = 1; step < 128; step <<= 1) {
        for (int t = tid; t < rows * 64; t += nthreads) {
            const int r = t >> 6, b = t & 63;
            const int i = ((b & ~(step - 1)) << 1) | (b & (step - 1));
            float *row = v + r * stride;
            const float a = row[i], c = row[i + step];
            row[i] = a + c;
            row[i + step] = a - c;
        }
        __syncthreads();
    }
    for (int t = tid; t < rows * 128; t += nthreads) v[(t >> 7) * stride + (t & 127)] *= 0.08838834764831844055f;
    __syncthreads();
}

// Value of lane lane ^ S (S = 1, 2, 4, 8) inside each row of 16 lanes, by DPP
// (row_ror:n gives lane i the value of lane (i - n) mod 16).
template <int S>
__device__ __forceinline__ float dpp_xor(float v) {
    const int iv = __float_as_int(v);
    if constexpr (S == 1) {
        return __int_as_float(__builtin_amdgcn_mov_dpp(iv, 0xB1, 0xF, 0xF, false));  // quad_perm 1,0,3,2
    } else if constexpr (S == 2) {
        return __int_as_float(__builtin_amdgcn_mov_dpp(iv, 0x4E, 0xF, 0xF, false));  // quad_perm 2,3,0,1
    } else if constexpr (S == 4) {
        // lanes 0-3 and 8-11 of the row (banks 0, 2) read lane + 4 (row_ror:12),
        // lanes 4-7 and 12-15 (banks 1, 3) read lane - 4 (row_ror:4)
        const int t = __builtin_amdgcn_update_dpp(iv, iv, 0x12C, 0xF, 0x5, false);
        return __int_as_float(__builtin_amdgcn_update_dpp(t, iv, 0x124, 0xF, 0xA, false));
    } else {
        static_assert(S == 8, "dpp_xor: S in 1, 2, 4, 8");
        return __int_as_float(__builtin_amdgcn_mov_dpp(iv, 0x128, 0xF, 0xF, false));  // row_ror:8
    }
}

// Layout of an H128 block spread over a 16-lane row with 8 consecutive elements
// per lane: lane l holds elements 8 b .. 8 b + 7 with b = h128_lane_block(l) =
// (l0 ^ l2, l1 ^ l2, l2, l3) in bits (an involution).  The cross-lane stages over
// block bits 1, 2, 4, 8 then pair lane l with l ^ 1, l ^ 2, l ^ 7 and l ^ 8, each
// one DPP read (xor 7 is row_half_mirror) where plain order needs two bank-masked
// reads and a copy for xor 4.
__device__ __forceinline__ int h128_lane_block(int l) { return l ^ (((l >> 2) & 1) * 3); }

// Value of the lane holding block b ^ S (S = 1, 2, 4, 8) in that layout.
template <int S>
__device__ __forceinline__ float dpp_block_xor(float v) {
    if constexpr (S == 4) {
        return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false));  // row_half_mirror
    } else {
        return dpp_xor<S>(v);
    }
}

// One cross-lane stage S of the block layout above on eight values per lane, in
// signed form: the butterfly sgn v + v' (sgn = -1 on the lane holding the upper
// block) equals sgn (v + sgn v'), so the stage keeps m = m + sgn dpp(m) and the
// caller multiplies the stage signs into one lane sign at the end.  Each value
// is one v_fmac_f32 whose first operand is the partner lane's register (DPP),
// where a separate DPP move and fma take two; the compiler does not fuse them.
// Every sum is rounded as in the unsigned form (round-to-nearest is
// sign-symmetric).  The s_nop gives the two wait states a DPP read needs after
// a VALU write of its register; inside the block each value's register was
// written eight instructions earlier.
template <int S>
__device__ __forceinline__ void dpp_block_stage8(float (&m)[8], float sgn) {
#define EXL3_FMAC8(CTL)                                                                                          \
    asm volatile("s_nop 1\n"                                                                                     \
                 "v_fmac_f32_dpp %0, %0, %8 " CTL " row_mask:0xf bank_mask:0xf\n"                                 \
                 "v_fmac_f32_dpp %1, %1, %8 " CTL " row_mask:0xf bank_mask:0xf\n"                                 \
                 "v_fmac_f32_dpp %2, %2, %8 " CTL " row_mask:0xf bank_mask:0xf\n"                                 \
                 "v_fmac_f32_dpp %3, %3, %8 " CTL " row_mask:0xf bank_mask:0xf\n"                                 \
                 "v_fmac_f32_dpp %4, %4, %8 " CTL " row_mask:0xf bank_mask:0xf\n"                                 \
                 "v_fmac_f32_dpp %5, %5, %8 " CTL " row_mask:0xf bank_mask:0xf\n"                                 \
                 "v_fmac_f32_dpp %6, %6, %8 " CTL " row_mask:0xf bank_mask:0xf\n"                                 \
                 "v_fmac_f32_dpp %7, %7, %8 " CTL " row_mask:0xf bank_mask:0xf"                                   \
                 : "+v"(m[0]), "+v"(m[1]), "+v"(m[2]), "+v"(m[3]), "+v"(m[4]), "+v"(m[5]), "+v"(m[6]), "+v"(m[7]) \
                 : "v"(sgn))
    if constexpr (S == 1) EXL3_FMAC8("quad_perm:[1,0,3,2]");
    else if constexpr (S == 2) EXL3_FMAC8("quad_perm:[2,3,0,1]");
    else if constexpr (S == 4) EXL3_FMAC8("row_half_mirror");
    else {
        static_assert(S == 8, "dpp_block_stage8: S in 1, 2, 4, 8");
        EXL3_FMAC8("row_ror:8");
    }
#undef EXL3_FMAC8
}

// H128 of one 128-block held by a wave: lane l owns element l in v0 and element
// l + 64 in v1.  Stages 1..32 pair lanes l and l ^ step, stage 64 pairs v0/v1;
// each butterfly is (a + b, a - b) with a the lower index, in the reference's
// stage order (src/exl3_codec.cpp:153-165), then the 1/sqrt(128) scale.  Lane
// exchanges are VALU only: DPP for xor 1..8 inside 16-lane rows, gfx950's
// v_permlane16_swap / v_permlane32_swap for xor 16 / 32; each butterfly is one
// fma with a +-1 lane sign, exact like a +- b.
//
// permlane{16,32}_swap(v, v) returns r0 = v with every upper half (odd 16-lane
// row, or lanes 32..63) replaced by the lower half next to it and r1 = v with
// every lower half replaced by the upper one: a lower lane reads own = r0,
// partner = r1, an upper lane partner = r0, own = r1, so r0 + sgn r1 is the
// butterfly on both.
template <int S>
__device__ __forceinline__ float lane_butterfly(float v, int lane) {
    const float sgn = (lane & S) ? -1.f : 1.f;  // upper element: partner - own
    if constexpr (S == 16 || S == 32) {
        const int iv = __float_as_int(v);
        const auto r = [&] {
            if constexpr (S == 16) return __builtin_amdgcn_permlane16_swap(iv, iv, false, false);
            else return __builtin_amdgcn_permlane32_swap(iv, iv, false, false);
        }();
        return __builtin_fmaf(__int_as_float(r[1]), sgn, __int_as_float(r[0]));
    } else {
        return __builtin_fmaf(v, sgn, dpp_xor<S>(v));
    }
}

template <int STEP>
__device__ __forceinline__ void h128_stage(float &v0, float &v1, int lane) {
    v0 = lane_butterfly<STEP>(v0, lane);
    v1 = lane_butterfly<STEP>(v1, lane);
}

__device__ __forceinline__ void h128_wave(float &v0, float &v1, int lane) {
    h128_stage<1>(v0, v1, lane);
    h128_stage<2>(v0, v1, lane);
    h128_stage<4>(v0, v1, lane);
    h128_stage<8>(v0, v1, lane);
    h128_stage<16>(v0, v1, lane);
    h128_stage<32>(v0, v1, lane);
    const float a = v0, b = v1;
    v0 = (a + b) * 0.08838834764831844055f;
    v1 = (a - b) * 0.08838834764831844055f;
}

// The same transform with lane l owning elements 2 l (e0) and 2 l + 1 (e1): the
// stride-1 butterfly is inside the lane, strides 2..64 pair lanes l and l ^ 1..32.
__device__ __forceinline__ void h128_pair(float &e0, float &e1, int lane) {
    const float a = e0, b = e1;
    e0 = a + b;
    e1 = a - b;
    h128_stage<1>(e0, e1, lane);
    h128_stage<2>(e0, e1, lane);
    h128_stage<4>(e0, e1, lane);
    h128_stage<8>(e0, e1, lane);
    h128_stage<16>(e0, e1, lane);
    h128_stage<32>(e0, e1, lane);
    e0 *= 0.08838834764831844055f;
    e1 *= 0.08838834764831844055f;
}

// ------------------------------------------------------------- chunk decode
// Chunk j (0..7) of a tile is its words [j K, j K + K): stream positions
// 32 j .. 32 j + 31.  The state of position 32 j + t is the window
// [K (t + 1) - 16, K (t + 1)) of stream bits counted from the chunk start (MSB
// of word j K first); the first windows reach back into the previous chunk's
// last word `prev` (chunk 7 for j = 0: the stream is cyclic,
// src/exl3_codec.cpp:103-108).  A window inside one word is a bit field of that
// word; a window across the boundary before word m is a bit field of
// xb[m] = alignbit(w[m - 1], w[m], 16), which spans the 16 bits on each side.
template <int K, int T>
__device__ __forceinline__ uint32_t chunk_state(const uint32_t (&w)[K], const uint32_t (&xb)[K]) {
    constexpr int a = K * (T + 1) - 16;  // window start, > -16
    constexpr int m = a >= 0 ? a / 32 : -1;
    if constexpr (a >= 0 && a + 16 <= 32 * (m + 1)) {
        return (w[m] >> (32 * (m + 1) - a - 16)) & 0xffffu;
    } else {
        constexpr int b = 32 * (m + 1);  // boundary crossed; xb[m + 1] spans [b - 16, b + 16)
        static_assert(m + 1 >= 0 && m + 1 < K, "window crosses an inner word boundary");
        return (xb[m + 1] >> (b - a)) & 0xffffu;
    }
}

// Positions 32 j + 8 q + e map to column j + 8 (e >> 2) and row
// 2 q + (e & 1) + 8 ((e >> 1) & 1) of the tile (src/exl3_codec.cpp:109-113), so the
// pair (8 q + 2 f, 8 q + 2 f + 1) is rows (2 q, 2 q + 1) + 8 (f & 1) of column
// j + 8 (f >> 1).  frag[f] packs q = 0..3: an MFMA A fragment of 8 consecutive
// rows (8 (f & 1) + 0..7) of one column, low half first.
template <int K, int CB, int F, int Q>
__device__ __forceinline__ uint32_t chunk_pair(const uint32_t (&w)[K], const uint32_t (&xb)[K]) {
    return codebook_pair<CB>(chunk_state<K, 8 * Q + 2 * F>(w, xb), chunk_state<K, 8 * Q + 2 * F + 1>(w, xb));
}
template <int K, int CB, int F>
__device__ __forceinline__ u4 chunk_frag(const uint32_t (&w)[K], const uint32_t (&xb)[K]) {
    return (u4){chunk_pair<K, CB, F, 0>(w, xb), chunk_pair<K, CB, F, 1>(w, xb), chunk_pair<K, CB, F, 2>(w, xb),
                chunk_pair<K, CB, F, 3>(w, xb)};
}
template <int K, int CB>
__device__ __forceinline__ void decode_chunk(const uint32_t (&w)[K], uint32_t prev, u4 (&frag)[4]) {
    uint32_t xb[K];
    xb[0] = __builtin_amdgcn_alignbit(prev, w[0], 16);
#pragma unroll
    for (int m = 1; m < K; ++m) xb[m] = __builtin_amdgcn_alignbit(w[m - 1], w[m], 16);
    frag[0] = chunk_frag<K, CB, 0>(w, xb);
    frag[1] = chunk_frag<K, CB, 1>(w, xb);
    frag[2] = chunk_frag<K, CB, 2>(w, xb);
    frag[3] = chunk_frag<K, CB, 3>(w, xb);
}

}  // namespace exl3dev
