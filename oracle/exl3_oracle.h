/*
 * exl3_oracle.h -- CPU restatement of the reference EXL3 codec and CPU layer.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or the timed CPU baseline).  The product library (libexl3_hip.so) never
 * links, loads or calls it.
 *
 * Every function cites the reference file:line whose behaviour it restates.
 * Return codes: 0 = success, ORC_EINVAL = the argument checks that the
 * reference expresses with std::invalid_argument / GGML_ASSERT failed.
 */
#ifndef EXL3_ORACLE_H
#define EXL3_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_OK 0
#define ORC_EINVAL 1

/* codebook ids: src/exl3_codec.h:8 (three_inst = 0, mcg = 1, mul1 = 2) */
#define ORC_CB_3INST 0u
#define ORC_CB_MCG 1u
#define ORC_CB_MUL1 2u

float orc_half_to_float(uint16_t h);                       /* src/exl3_codec.cpp:21-38 */
uint16_t orc_float_to_half(float f);                       /* src/exl3_codec.cpp:40-66 */
uint16_t orc_decode_codebook(uint16_t state, unsigned cb); /* src/exl3_codec.cpp:68-86 */

/* one 16x16 tile of 16*bits little-endian u16 -> row-major fp16 bits.
 * src/exl3_codec.cpp:92-115 */
int orc_decode_tile(const uint16_t *packed, unsigned bits, unsigned cb, uint16_t *row_major);

/* upstream tile grid [k/16][n/16][16*bits] -> row-major [k][count] fp16.
 * src/exl3_codec.cpp:117-145 */
int orc_decode_inner_slice(const uint16_t *packed, size_t k, size_t n, size_t first_column,
                           size_t column_count, unsigned bits, unsigned cb, uint16_t *out);
int orc_decode_inner(const uint16_t *packed, size_t k, size_t n, unsigned bits, unsigned cb,
                     uint16_t *out);

/* in-place orthonormal H128 over each 128-block.  src/exl3_codec.cpp:147-167 */
int orc_hadamard128(float *values, size_t count);

/* original-basis weight diag(su) H W H diag(sv), [k][count] fp16.
 * src/exl3_codec.cpp:169-204 */
int orc_reconstruct_slice(const uint16_t *packed, const uint16_t *su, const uint16_t *sv,
                          size_t k, size_t n, size_t first_column, size_t column_count,
                          unsigned bits, unsigned cb, uint16_t *out);
int orc_reconstruct(const uint16_t *packed, const uint16_t *su, const uint16_t *sv, size_t k,
                    size_t n, unsigned bits, unsigned cb, uint16_t *out);

/* ---- 128x128 group-record layout (include/exl3-block.h:5-14,34-39) ---- */

/* GET_ROWS on records (src/exl3-ggml.cpp:19-49): out[r][0..k) (row stride
 * out_stride floats) = column ids[r] of the original-basis weight, each record's
 * 128x128 reconstruct rounded to fp16 and widened; ORC_EINVAL on an id outside
 * [0, n) (the reference asserts). */
int orc_get_rows(const void *records, unsigned bits, unsigned cb, size_t k, size_t n, const int32_t *ids,
                 size_t count, float *out, size_t out_stride);
size_t orc_group_bytes(unsigned bits); /* include/exl3-block.h:14 */

/* upstream tiles + su + sv -> records, tests/test-exl3-graph.cpp:37-45 and
 * tools/export_native_gguf.py:27-36 */
int orc_pack_records(const uint16_t *packed, const uint16_t *su, const uint16_t *sv, size_t k,
                     size_t n, unsigned bits, void *records);

/* records -> row-major [k][n] fp16 (decode_inner over the record layout) */
int orc_decode_records(const void *records, size_t k, size_t n, unsigned bits, unsigned cb,
                       uint16_t *out);

/* 1 if every su/sv value of every record is finite, 0 otherwise, -1 on a
 * size that is not a whole number of records.  patches/llama-exl3.patch:327-338 */
int orc_validate_records(const void *records, size_t nbytes, unsigned bits);

/* CPU reference layer: ggml_exl3_mul_mat, src/exl3-ggml.cpp:51-92.
 * x: rows of k values, fp16 (x_is_f16 = 1) or fp32, row stride in bytes.
 * y: rows of n fp32 values, row stride in bytes.
 * nthreads >= 1 worker threads partition the 128-column groups exactly as
 * ggml does (nb = ith; nb += nth).  cb is mul1 in the reference (:78); other
 * codebooks are accepted for testing. */
int orc_mul_mat(const void *records, unsigned bits, unsigned cb, size_t k, size_t n,
                const void *x, int x_is_f16, size_t rows, size_t x_stride_bytes, float *y,
                size_t y_stride_bytes, unsigned nthreads);

/* Same, but only for column groups [nb_begin, nb_end): used to time a bounded
 * sample of a large layer. */
int orc_mul_mat_groups(const void *records, unsigned bits, unsigned cb, size_t k, size_t n,
                       const void *x, int x_is_f16, size_t rows, size_t x_stride_bytes,
                       float *y, size_t y_stride_bytes, unsigned nthreads, size_t nb_begin,
                       size_t nb_end);

/* The DSP service's layer exl3_iface_matmul, src/hexagon/exl3_service.c:265-305:
 * the same math as orc_mul_mat on the upstream tile layout [k/16][n/16][16 bits]
 * with separate su[k] / sv[n] (fp16), fp32 x (batch x k) and y (batch x n),
 * accumulated in the service's loop order rk -> cn -> row -> col -> b (:248-261).
 * Argument checks of :270-273 (batch <= 8, k * n <= 64 Mi) -> ORC_EINVAL. */
int orc_iface_matmul(unsigned bits, unsigned cb, size_t k, size_t n, size_t batch, const uint16_t *packed,
                     const uint16_t *suh, const uint16_t *svh, const float *x, float *y);

#ifdef __cplusplus
}
#endif

#endif
