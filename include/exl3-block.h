/*
 * exl3-block.h -- the 128x128 EXL3 group-record layout.
 *
 * Same names, type ids, byte layout and helper functions as the reference's
 * include/exl3-block.h:1-50, so records written for the reference's ggml types
 * 43/44/45 are consumed unchanged by the HIP path and code written against the
 * reference header (its codec test, its ggml glue) compiles against this one.
 *
 * A record covers 128 input rows (k) x 128 output columns (n):
 *   [ 64 trellis tiles of 32*bits bytes, tile (r, c) at byte (8 r + c) * 32 * bits ]
 *   [ su[128] fp16 : input scales of this record's 128 rows    ]
 *   [ sv[128] fp16 : output scales of this record's 128 columns ]
 * Record (nb, kb) of a k x n matrix starts at byte (nb * (k / 128) + kb) * exl3_group_bytes(bits),
 * i.e. records are column-group-major, so a 128-column group is one contiguous run.
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#define EXL3_TYPE_4 43
#define EXL3_TYPE_6 44
#define EXL3_TYPE_8 45
#define EXL3_GROUP_DIM 128
/* bytes of zero padding behind a decoded group in the DSP's scratch (include/exl3-block.h:9) */
#define EXL3_DECODE_PAD_BYTES 128

/* ggml type id -> bits per weight (0 if not an EXL3 type); include/exl3-block.h:11-13 */
static inline unsigned exl3_type_bits(unsigned type) {
    switch (type) {
    case EXL3_TYPE_4: return 4;
    case EXL3_TYPE_6: return 6;
    case EXL3_TYPE_8: return 8;
    default: return 0;
    }
}

/* bytes of one 128x128 record: 64 tiles of 32*bits bytes + 128 su + 128 sv halves;
 * include/exl3-block.h:14 */
static inline size_t exl3_group_bytes(unsigned bits) { return (size_t) 2048 * bits + 512; }

/*
 * Hexagon VTCM scratch planners (include/exl3-block.h:15-33).  They size the DSP
 * workers' scratch memory of the reference's HTP op and mean nothing for the GPU
 * kernels, which take a device workspace sized by exl3_hip_mul_mat_workspace_bytes
 * instead.  They are kept, with the reference's integer results, so callers and
 * tests written against the reference header keep compiling and computing the
 * same plans.
 *
 * Per-worker scratch of the HVX path for `rows` activation rows: one decoded
 * 128x128 fp16 group (32 KiB) plus its decode padding, 512 bytes of fp32 output
 * per row, one packed group and 640 bytes of vectors.
 */
static inline size_t exl3_thread_bytes(unsigned bits, size_t rows) {
    const size_t decoded_group = (size_t) 128 * 128 * 2;
    const size_t out_rows = rows * 128 * 4;
    return decoded_group + EXL3_DECODE_PAD_BYTES + out_rows + exl3_group_bytes(bits) + 640;
}

/* Shared scratch of the HMX path beyond the activations: 64 bytes per input
 * feature, 256 + 4096 bytes of tables and 10 KiB per worker (8 KiB + 2 KiB). */
static inline size_t exl3_hmx_extra(size_t k, unsigned threads) {
    return k * 64 + 256 + 4096 + (size_t) threads * (8192 + 2048);
}

/* round up to the HMX's 2 KiB alignment */
static inline size_t exl3_hmx_align2k(size_t bytes) { return (bytes + 2047) & ~(size_t) 2047; }

/* Byte offset where the HMX path's per-call tables start: the fp32 activations
 * (rows x k x 4 bytes), rounded up to 2 KiB. */
static inline size_t exl3_hmx_activation_offset(size_t k, size_t rows) { return exl3_hmx_align2k(rows * k * 4); }

/* Per-worker HMX scratch: the HVX worker scratch rounded up to 2 KiB, then an
 * 8 KiB HMX output tile. */
static inline size_t exl3_hmx_thread_bytes(unsigned bits, size_t rows) {
    return exl3_hmx_align2k(exl3_thread_bytes(bits, rows)) + 8192;
}

/* Shared HMX prefix: activations, then 64 bytes per feature plus 256, rounded
 * up to 2 KiB. */
static inline size_t exl3_hmx_prefix_bytes(size_t k, size_t rows) {
    return exl3_hmx_align2k(exl3_hmx_activation_offset(k, rows) + k * 64 + 256);
}

/* Activation rows one HTP call processes within vtcm_size bytes: what is left
 * after every worker's empty scratch, divided by the bytes a row costs (k fp32
 * activations + 512 output bytes per worker), capped at 32; 0 when nothing fits
 * or there is no worker or no input feature. */
static inline size_t exl3_row_chunk(unsigned bits, size_t k, unsigned threads, size_t vtcm_size) {
    if (threads == 0 || k == 0) return 0;
    const size_t fixed = (size_t) threads * exl3_thread_bytes(bits, 0);
    if (vtcm_size <= fixed) return 0;
    const size_t per_row = k * 4 + (size_t) threads * 512;
    const size_t fit = (vtcm_size - fixed) / per_row;
    return fit > 32 ? 32 : fit;
}

/* the record's su / sv vectors; include/exl3-block.h:34-39 */
static inline const uint16_t * exl3_group_su(const void * group, unsigned bits) {
    return (const uint16_t *) ((const unsigned char *) group + (size_t) 2048 * bits);
}
static inline const uint16_t * exl3_group_sv(const void * group, unsigned bits) {
    return (const uint16_t *) ((const unsigned char *) group + (size_t) 2048 * bits + 256);
}

/*
 * The reference's ggml CPU ops (include/exl3-block.h:41-50).  They are defined
 * by the engine-side glue that owns the ggml types (in the reference,
 * src/exl3-ggml.cpp), not by libexl3_hip.so; a HIP backend binds
 * exl3_hip_mul_mat / exl3_hip_get_rows (exl3_hip.h) in their place.  Declared
 * here so that translation units written against the reference header compile.
 */
struct ggml_compute_params;
struct ggml_tensor;
#ifdef __cplusplus
extern "C" {
#endif
void ggml_exl3_mul_mat(const struct ggml_compute_params * params, struct ggml_tensor * dst);
void ggml_exl3_get_rows(const struct ggml_compute_params * params, struct ggml_tensor * dst);
#ifdef __cplusplus
}
#endif
