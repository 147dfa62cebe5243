/*
 * exl3_oracle.c -- CPU restatement of the reference EXL3 codec (src/exl3_codec.cpp),
 * the 128x128 group-record layout (include/exl3-block.h) and the CPU layer
 * ggml_exl3_mul_mat (src/exl3-ggml.cpp:51-92).
 *
 * TEST INFRASTRUCTURE ONLY: this is the checker that the HIP path is compared
 * against, and the CPU baseline that bench.py times.  The product library does
 * not link or call it.
 *
 * Pinning (how each function is held to the reference, not just restated):
 *   - orc_half_to_float / orc_float_to_half: all 2^16 halves and all 2^32
 *     floats compared against the compiled reference codec (oracle/check_ref.c),
 *     plus the reference's own known answers (tests/test_codec.cpp:58-65).
 *   - orc_decode_codebook: all 3 x 65536 states against the compiled reference
 *     and the mul1 closed form (tests/test_codec.cpp:16-31).
 *   - orc_decode_tile / decode_inner(_slice): golden tiles and 256x384 matrices
 *     for bits 1..8 x 3 codebooks produced by the compiled reference codec
 *     (tests/golden/), zero-ring (tests/test_codec.cpp:72-80), rejects (:81-88).
 *   - orc_hadamard128: Sylvester matrix closed form, involution
 *     (tests/test_codec.cpp:66-71), compiled reference on random vectors.
 *   - orc_reconstruct(_slice): compiled reference, bit for bit; slice == full
 *     (tools/exl3_verify.cpp:57-66).
 *   - orc_pack_records / orc_decode_records: record offsets re-derived from
 *     include/exl3-block.h and checked against decode_inner of the tile grid.
 *   - orc_get_rows: column ids[r] of orc_reconstruct over the whole matrix, and
 *     the zero-trellis closed form (tests/test_model_reader.cpp:51-56).
 *   - orc_mul_mat: float64 x . reconstruct(W) with the compiled reference
 *     reconstruct, NMSE < 1e-5 (the gate of tests/test-exl3-graph.cpp:100-104),
 *     and planted-mistake tests showing that gate catches a dropped su/sv, a
 *     missing Hadamard and a transposed tile.
 */
#include "exl3_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ fp16 */

/* src/exl3_codec.cpp:21-38: binary16 -> binary32, exact. */
float orc_half_to_float(uint16_t h)
{
    const uint32_t negative = h & 0x8000u;
    const uint32_t field = (h >> 10) & 0x1fu;
    const uint32_t frac = h & 0x3ffu;
    if (field == 0) {
        /* zero and subnormals: frac * 2^-24 */
        const float v = ldexpf((float)frac, -24);
        return negative ? -v : v;
    }
    const uint32_t e32 = field == 0x1fu ? 0xffu : field + (127u - 15u);
    const uint32_t word = (negative << 16) | (e32 << 23) | (frac << 13);
    float out;
    memcpy(&out, &word, sizeof out);
    return out;
}

/* round-half-to-even of v / 2^s, s >= 1 */
static uint32_t rne_shift(uint32_t v, unsigned s)
{
    const uint32_t kept = v >> s;
    const uint32_t dropped = v & ((1u << s) - 1u);
    const uint32_t half = 1u << (s - 1u);
    const int up = dropped > half || (dropped == half && (kept & 1u));
    return kept + (uint32_t)up;
}

/* src/exl3_codec.cpp:40-66: binary32 -> binary16, round half to even,
 * subnormal results, overflow to infinity, NaN -> quiet 0x7e00. */
uint16_t orc_float_to_half(float f)
{
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t e = (u >> 23) & 0xffu;
    const uint32_t m = u & 0x7fffffu;
    if (e == 0xffu) return (uint16_t)(sign | (m ? 0x7e00u : 0x7c00u));
    if (e >= 143u) return (uint16_t)(sign | 0x7c00u);   /* |f| >= 2^16 */
    if (e <= 101u) return sign;                         /* |f| <  2^-25 */
    if (e <= 112u) {
        /* half subnormal: |f| / 2^-24 = (1.m) * 2^(e - 103) */
        return (uint16_t)(sign | rne_shift(m | 0x800000u, 126u - e));
    }
    /* normal: rounding carry may ripple into the exponent (and to 0x7c00) */
    return (uint16_t)(sign | (((e - 112u) << 10) + rne_shift(m, 13u)));
}

/* ------------------------------------------------------------- codebooks */

static unsigned byte_sum(uint32_t v)
{
    return (v & 0xffu) + ((v >> 8) & 0xffu) + ((v >> 16) & 0xffu) + (v >> 24);
}

/* src/exl3_codec.cpp:68-86.
 * mul1: the reference evaluates fma(half(0x6400 + s), half(0x1eee), half(0xc931))
 * in binary32 and rounds once to binary16; that binary32 value is exact and
 * equals (1774 s - 905216) / 2^18 (tests/test_codec.cpp:16-31), which is the
 * form used here.
 * mcg / 3inst: P' = (P & 0x8fff8fff) ^ 0x3b603b60 and the result is the
 * binary16 rounding of half(P'.lo) + half(P'.hi) (the binary32 sum is exact). */
uint16_t orc_decode_codebook(uint16_t state, unsigned cb)
{
    const uint32_t s = state;
    uint32_t p;
    switch (cb) {
    case ORC_CB_MUL1: {
        const int sum = (int)byte_sum(s * 0x83dcd12du);
        const float exact = (float)(1774 * sum - 905216) / 262144.0f;
        return orc_float_to_half(exact);
    }
    case ORC_CB_MCG:
        p = s * 0xcbac1fedu;
        break;
    case ORC_CB_3INST:
        p = s * 89226354u + 64248484u;
        break;
    default:
        return 0x7e00u;
    }
    p = (p & 0x8fff8fffu) ^ 0x3b603b60u;
    const float sum = orc_half_to_float((uint16_t)(p & 0xffffu)) + orc_half_to_float((uint16_t)(p >> 16));
    return orc_float_to_half(sum);
}

/* the reference decodes through a precomputed 3 x 65536 table
 * (src/exl3_codec.cpp:94-100); the same is done here for speed */
static uint16_t g_table[3][65536];
static pthread_once_t g_table_once = PTHREAD_ONCE_INIT;

static void build_tables(void)
{
    for (unsigned cb = 0; cb < 3; ++cb)
        for (uint32_t st = 0; st < 65536u; ++st) g_table[cb][st] = orc_decode_codebook((uint16_t)st, cb);
}

static const uint16_t *codebook_table(unsigned cb)
{
    pthread_once(&g_table_once, build_tables);
    return g_table[cb];
}

/* ------------------------------------------------------------ tile decode */

static int valid_rate(unsigned bits, unsigned cb) { return bits >= 1u && bits <= 8u && cb <= 2u; }

/* u32 word i of a tile stream: little-endian pair of u16 (src/exl3_codec.cpp:88-90) */
static uint32_t stream_word(const uint16_t *t, unsigned i)
{
    return (uint32_t)t[2u * i] | ((uint32_t)t[2u * i + 1u] << 16);
}

/* Trellis state of position p: the 16-bit MSB-first window of the cyclic
 * 256*bits-bit stream that ends (exclusive) at bit (p + 1) * bits.
 * src/exl3_codec.cpp:102-108. */
static uint16_t tile_state(const uint16_t *t, unsigned bits, unsigned p)
{
    const unsigned nbits = 256u * bits, nwords = 8u * bits;
    const unsigned first = ((p + 1u) * bits + nbits - 16u) % nbits;
    const unsigned w = first / 32u, off = first % 32u;
    const uint64_t pair = ((uint64_t)stream_word(t, w) << 32) | stream_word(t, (w + 1u) % nwords);
    return (uint16_t)(pair >> (48u - off));
}

/* Position p = 8 * lane + e -> (row, col) of the 16x16 tile, the upstream
 * tensor-core fragment order.  src/exl3_codec.cpp:109-113. */
static void tile_coord(unsigned p, unsigned *row, unsigned *col)
{
    const unsigned lane = p >> 3, e = p & 7u;
    *row = 2u * (lane & 3u) + (e & 1u) + 8u * ((e >> 1) & 1u);
    *col = (lane >> 2) + 8u * ((e >> 2) & 1u);
}

static void decode_tile_unchecked(const uint16_t *packed, unsigned bits, const uint16_t *table,
                                  uint16_t *dst, size_t dst_stride)
{
    for (unsigned p = 0; p < 256u; ++p) {
        unsigned r, c;
        tile_coord(p, &r, &c);
        dst[r * dst_stride + c] = table[tile_state(packed, bits, p)];
    }
}

/* src/exl3_codec.cpp:92-115 */
int orc_decode_tile(const uint16_t *packed, unsigned bits, unsigned cb, uint16_t *row_major)
{
    if (!valid_rate(bits, cb)) return ORC_EINVAL;
    decode_tile_unchecked(packed, bits, codebook_table(cb), row_major, 16);
    return ORC_OK;
}

/* src/exl3_codec.cpp:117-121 */
static int valid_shape(size_t k, size_t n, size_t multiple)
{
    return k && n && k % multiple == 0 && n % multiple == 0 && k <= SIZE_MAX / n;
}

/* src/exl3_codec.cpp:128-145 */
int orc_decode_inner_slice(const uint16_t *packed, size_t k, size_t n, size_t first_column,
                           size_t column_count, unsigned bits, unsigned cb, uint16_t *out)
{
    if (!valid_rate(bits, cb) || !valid_shape(k, n, 16)) return ORC_EINVAL;
    if (!column_count || first_column % 16 || column_count % 16 || first_column > n ||
        column_count > n - first_column)
        return ORC_EINVAL;
    const uint16_t *table = codebook_table(cb);
    const size_t tiles_per_row = n / 16, tile_u16 = 16u * bits;
    for (size_t rk = 0; rk < k / 16; ++rk)
        for (size_t cn = 0; cn < column_count / 16; ++cn) {
            const uint16_t *src = packed + (rk * tiles_per_row + first_column / 16 + cn) * tile_u16;
            decode_tile_unchecked(src, bits, table, out + rk * 16 * column_count + cn * 16, column_count);
        }
    return ORC_OK;
}

int orc_decode_inner(const uint16_t *packed, size_t k, size_t n, unsigned bits, unsigned cb,
                     uint16_t *out)
{
    return orc_decode_inner_slice(packed, k, n, 0, n, bits, cb, out);
}

/* ---------------------------------------------------------------- H128 */

#define ORC_H128_SCALE 0.08838834764831844055f /* 1/sqrt(128) as binary32 0x3db504f3 */

static void h128_block(float *v)
{
    for (unsigned step = 1; step < 128u; step <<= 1)
        for (unsigned i = 0; i < 128u; ++i)
            if (!(i & step)) {
                const float a = v[i], b = v[i + step];
                v[i] = a + b;
                v[i + step] = a - b;
            }
    for (unsigned i = 0; i < 128u; ++i) v[i] *= ORC_H128_SCALE;
}

/* src/exl3_codec.cpp:147-167 */
int orc_hadamard128(float *values, size_t count)
{
    if (count % 128u) return ORC_EINVAL;
    for (size_t b = 0; b < count; b += 128u) h128_block(values + b);
    return ORC_OK;
}

/* ---------------------------------------------------------- reconstruct */

/* src/exl3_codec.cpp:174-204: per 128x128 block, H over each row (along n),
 * then H over each column (along k), then binary32 (w * su) * sv rounded to
 * binary16. */
int orc_reconstruct_slice(const uint16_t *packed, const uint16_t *su, const uint16_t *sv,
                          size_t k, size_t n, size_t first_column, size_t column_count,
                          unsigned bits, unsigned cb, uint16_t *out)
{
    if (!valid_shape(k, n, 128) || first_column % 128 || column_count % 128) return ORC_EINVAL;
    const int rc = orc_decode_inner_slice(packed, k, n, first_column, column_count, bits, cb, out);
    if (rc) return rc;
    float *blk = (float *)malloc(128u * 128u * sizeof(float));
    if (!blk) return ORC_EINVAL;
    float col[128];
    for (size_t rk = 0; rk < k; rk += 128)
        for (size_t cn = 0; cn < column_count; cn += 128) {
            for (size_t r = 0; r < 128; ++r)
                for (size_t c = 0; c < 128; ++c)
                    blk[r * 128 + c] = orc_half_to_float(out[(rk + r) * column_count + cn + c]);
            for (size_t r = 0; r < 128; ++r) h128_block(blk + r * 128);
            for (size_t c = 0; c < 128; ++c) {
                for (size_t r = 0; r < 128; ++r) col[r] = blk[r * 128 + c];
                h128_block(col);
                const float s_out = orc_half_to_float(sv[first_column + cn + c]);
                for (size_t r = 0; r < 128; ++r) {
                    const float scaled = col[r] * orc_half_to_float(su[rk + r]);
                    out[(rk + r) * column_count + cn + c] = orc_float_to_half(scaled * s_out);
                }
            }
        }
    free(blk);
    return ORC_OK;
}

int orc_reconstruct(const uint16_t *packed, const uint16_t *su, const uint16_t *sv, size_t k,
                    size_t n, unsigned bits, unsigned cb, uint16_t *out)
{
    return orc_reconstruct_slice(packed, su, sv, k, n, 0, n, bits, cb, out);
}

/* src/exl3-ggml.cpp:19-49 (ggml_exl3_get_rows): out[r][128 kb + i] =
 * float(reconstruct of record (ids[r] / 128, kb) as a 128x128 matrix)[i][ids[r] % 128]. */
int orc_get_rows(const void *records, unsigned bits, unsigned cb, size_t k, size_t n, const int32_t *ids,
                 size_t count, float *out, size_t out_stride)
{
    if (!valid_rate(bits, cb) || !valid_shape(k, n, 128) || out_stride < k) return ORC_EINVAL;
    for (size_t r = 0; r < count; ++r)
        if (ids[r] < 0 || (size_t)ids[r] >= n) return ORC_EINVAL;
    uint16_t *dec = (uint16_t *)malloc(128u * 128u * sizeof(uint16_t));
    if (!dec) return ORC_EINVAL;
    const size_t gb = orc_group_bytes(bits);
    for (size_t r = 0; r < count; ++r) {
        const size_t id = (size_t)ids[r];
        for (size_t kb = 0; kb < k / 128; ++kb) {
            const unsigned char *g = (const unsigned char *)records + ((id / 128) * (k / 128) + kb) * gb;
            const int rc = orc_reconstruct((const uint16_t *)g, (const uint16_t *)(g + 2048u * bits),
                                           (const uint16_t *)(g + 2048u * bits + 256u), 128, 128, bits, cb, dec);
            if (rc) {
                free(dec);
                return rc;
            }
            for (size_t i = 0; i < 128; ++i) out[r * out_stride + kb * 128 + i] = orc_half_to_float(dec[i * 128 + id % 128]);
        }
    }
    free(dec);
    return ORC_OK;
}

/* --------------------------------------------------------- record layout */

/* include/exl3-block.h:14: 64 tiles of 32*bits bytes, then su[128], sv[128] fp16 */
size_t orc_group_bytes(unsigned bits) { return 2048u * (size_t)bits + 512u; }

static size_t record_offset(size_t nb, size_t kb, size_t k, unsigned bits)
{
    return (nb * (k / 128) + kb) * orc_group_bytes(bits);
}

/* tests/test-exl3-graph.cpp:37-45, tools/export_native_gguf.py:27-36:
 * record (nb, kb), tile (r, c) = upstream tile (8 kb + r, 8 nb + c) */
int orc_pack_records(const uint16_t *packed, const uint16_t *su, const uint16_t *sv, size_t k,
                     size_t n, unsigned bits, void *records)
{
    if (bits < 1 || bits > 8 || !valid_shape(k, n, 128)) return ORC_EINVAL;
    const size_t tile_bytes = 32u * bits;
    unsigned char *base = (unsigned char *)records;
    for (size_t nb = 0; nb < n / 128; ++nb)
        for (size_t kb = 0; kb < k / 128; ++kb) {
            unsigned char *g = base + record_offset(nb, kb, k, bits);
            for (size_t r = 0; r < 8; ++r)
                for (size_t c = 0; c < 8; ++c) {
                    const size_t upstream_tile = (kb * 8 + r) * (n / 16) + nb * 8 + c;
                    memcpy(g + (r * 8 + c) * tile_bytes, packed + upstream_tile * 16u * bits, tile_bytes);
                }
            memcpy(g + 2048u * bits, su + kb * 128, 256);
            memcpy(g + 2048u * bits + 256u, sv + nb * 128, 256);
        }
    return ORC_OK;
}

int orc_decode_records(const void *records, size_t k, size_t n, unsigned bits, unsigned cb,
                       uint16_t *out)
{
    if (!valid_rate(bits, cb) || !valid_shape(k, n, 128)) return ORC_EINVAL;
    const uint16_t *table = codebook_table(cb);
    const unsigned char *base = (const unsigned char *)records;
    for (size_t nb = 0; nb < n / 128; ++nb)
        for (size_t kb = 0; kb < k / 128; ++kb) {
            const unsigned char *g = base + record_offset(nb, kb, k, bits);
            for (size_t r = 0; r < 8; ++r)
                for (size_t c = 0; c < 8; ++c) {
                    const uint16_t *tile = (const uint16_t *)(g + (r * 8 + c) * 32u * bits);
                    decode_tile_unchecked(tile, bits, table, out + (kb * 128 + r * 16) * n + nb * 128 + c * 16, n);
                }
        }
    return ORC_OK;
}

/* patches/llama-exl3.patch:327-338 (ggml_validate_row_data for EXL3 types) */
int orc_validate_records(const void *records, size_t nbytes, unsigned bits)
{
    const size_t gb = orc_group_bytes(bits);
    if (bits < 1 || bits > 8 || nbytes % gb) return -1;
    const unsigned char *base = (const unsigned char *)records;
    for (size_t off = 0; off < nbytes; off += gb) {
        const uint16_t *scales = (const uint16_t *)(base + off + 2048u * bits);
        for (unsigned i = 0; i < 256u; ++i)
            if ((scales[i] & 0x7c00u) == 0x7c00u) return 0;
    }
    return 1;
}

/* ------------------------------------------------------------ CPU layer */

struct mm_job {
    const unsigned char *records;
    unsigned bits;
    const uint16_t *table;
    size_t k, n, rows;
    const unsigned char *x;
    int x_is_f16;
    size_t x_stride;
    unsigned char *y;
    size_t y_stride;
    unsigned ith, nth;
    size_t nb_begin, nb_end;
    int failed;
};

static float load_x(const struct mm_job *j, size_t r, size_t i)
{
    const unsigned char *row = j->x + r * j->x_stride;
    if (j->x_is_f16) {
        uint16_t h;
        memcpy(&h, row + i * 2, 2);
        return orc_half_to_float(h);
    }
    float v;
    memcpy(&v, row + i * 4, 4);
    return v;
}

/* One ggml worker (ith of nth).  src/exl3-ggml.cpp:51-92:
 *   every worker builds xh[r] = H128(x[r] * su) for all rows, with su taken
 *   from record (0, kb) (:60-73);
 *   worker ith owns column groups nb = ith, ith + nth, ... (:74);
 *   result[r][j] += xh[r][128 kb + i] * W_kb[i][j] in binary32, loop order
 *   kb -> i -> j -> r (:76-82);
 *   y[r][128 nb + j] = H128(result[r])[j] * sv[j], sv from record (nb, 0)
 *   (:84-90). */
static void *mm_worker(void *arg)
{
    struct mm_job *j = (struct mm_job *)arg;
    const size_t k = j->k, rows = j->rows, kbs = k / 128, gb = orc_group_bytes(j->bits);
    float *xh = (float *)malloc(rows * k * sizeof(float));
    float *acc = (float *)malloc(rows * 128 * sizeof(float));
    uint16_t *w = (uint16_t *)malloc(128 * 128 * sizeof(uint16_t));
    if (!xh || !acc || !w) {
        j->failed = 1;
        free(xh);
        free(acc);
        free(w);
        return NULL;
    }
    for (size_t kb = 0; kb < kbs; ++kb) {
        const uint16_t *su = (const uint16_t *)(j->records + kb * gb + 2048u * j->bits);
        for (size_t r = 0; r < rows; ++r) {
            float *dst = xh + r * k + kb * 128;
            for (size_t i = 0; i < 128; ++i) dst[i] = load_x(j, r, kb * 128 + i) * orc_half_to_float(su[i]);
            h128_block(dst);
        }
    }
    size_t first = j->nb_begin;
    while (first % j->nth != j->ith) ++first; /* same residue class as nb = ith; nb += nth */
    for (size_t nb = first; nb < j->nb_end; nb += j->nth) {
        memset(acc, 0, rows * 128 * sizeof(float));
        for (size_t kb = 0; kb < kbs; ++kb) {
            const unsigned char *g = j->records + (nb * kbs + kb) * gb;
            for (size_t r8 = 0; r8 < 8; ++r8)
                for (size_t c8 = 0; c8 < 8; ++c8)
                    decode_tile_unchecked((const uint16_t *)(g + (r8 * 8 + c8) * 32u * j->bits), j->bits, j->table,
                                          w + r8 * 16 * 128 + c8 * 16, 128);
            for (size_t i = 0; i < 128; ++i)
                for (size_t c = 0; c < 128; ++c) {
                    const float wv = orc_half_to_float(w[i * 128 + c]);
                    for (size_t r = 0; r < rows; ++r) acc[r * 128 + c] += xh[r * k + kb * 128 + i] * wv;
                }
        }
        const uint16_t *sv = (const uint16_t *)(j->records + nb * kbs * gb + 2048u * j->bits + 256u);
        for (size_t r = 0; r < rows; ++r) {
            h128_block(acc + r * 128);
            float *yrow = (float *)(j->y + r * j->y_stride);
            for (size_t c = 0; c < 128; ++c) yrow[nb * 128 + c] = acc[r * 128 + c] * orc_half_to_float(sv[c]);
        }
    }
    free(xh);
    free(acc);
    free(w);
    return NULL;
}

int orc_mul_mat_groups(const void *records, unsigned bits, unsigned cb, size_t k, size_t n,
                       const void *x, int x_is_f16, size_t rows, size_t x_stride_bytes,
                       float *y, size_t y_stride_bytes, unsigned nthreads, size_t nb_begin,
                       size_t nb_end)
{
    /* src/exl3-ggml.cpp:56-57 */
    if (!valid_rate(bits, cb) || !valid_shape(k, n, 128) || !rows || !nthreads) return ORC_EINVAL;
    if (nb_begin > nb_end || nb_end > n / 128) return ORC_EINVAL;
    const size_t xe = x_is_f16 ? 2u : 4u;
    if (x_stride_bytes < k * xe || y_stride_bytes < n * 4u) return ORC_EINVAL;
    struct mm_job *jobs = (struct mm_job *)calloc(nthreads, sizeof *jobs);
    pthread_t *tids = (pthread_t *)calloc(nthreads, sizeof *tids);
    if (!jobs || !tids) {
        free(jobs);
        free(tids);
        return ORC_EINVAL;
    }
    const uint16_t *table = codebook_table(cb);
    for (unsigned t = 0; t < nthreads; ++t) {
        jobs[t] = (struct mm_job){(const unsigned char *)records, bits, table, k, n, rows,
                                  (const unsigned char *)x, x_is_f16, x_stride_bytes,
                                  (unsigned char *)y, y_stride_bytes, t, nthreads, nb_begin, nb_end, 0};
    }
    int failed = 0;
    if (nthreads == 1) {
        mm_worker(&jobs[0]);
    } else {
        unsigned started = 0;
        for (; started < nthreads; ++started)
            if (pthread_create(&tids[started], NULL, mm_worker, &jobs[started])) break;
        for (unsigned t = 0; t < started; ++t) pthread_join(tids[t], NULL);
        if (started != nthreads) failed = 1;
    }
    for (unsigned t = 0; t < nthreads; ++t) failed |= jobs[t].failed;
    free(jobs);
    free(tids);
    return failed ? ORC_EINVAL : ORC_OK;
}

int orc_mul_mat(const void *records, unsigned bits, unsigned cb, size_t k, size_t n,
                const void *x, int x_is_f16, size_t rows, size_t x_stride_bytes, float *y,
                size_t y_stride_bytes, unsigned nthreads)
{
    return orc_mul_mat_groups(records, bits, cb, k, n, x, x_is_f16, rows, x_stride_bytes, y,
                              y_stride_bytes, nthreads, 0, n / 128);
}

/* ------------------------------------------------ DSP service layer */

/* src/hexagon/exl3_service.c:265-305 (exl3_iface_matmul): xh[b] = H128(x[b] * su) (:280-286),
 * result[b][16 cn + col] += xh[b][16 rk + row] * W[16 rk + row][16 cn + col] in
 * binary32, loop order rk -> cn -> row -> col -> b (:248-261, tiles decoded by the
 * codec's formula, :67-86), then y[b] = H128(result[b]) * sv (:297-300). */
int orc_iface_matmul(unsigned bits, unsigned cb, size_t k, size_t n, size_t batch, const uint16_t *packed,
                     const uint16_t *suh, const uint16_t *svh, const float *x, float *y)
{
    if (!valid_rate(bits, cb) || !valid_shape(k, n, 128) || !batch || batch > 8 ||
        (uint64_t)k * n > 64u * 1024u * 1024u)
        return ORC_EINVAL;
    const uint16_t *table = codebook_table(cb);
    float *xh = (float *)malloc(batch * k * sizeof(float));
    float *result = (float *)calloc(batch * n, sizeof(float));
    if (!xh || !result) {
        free(xh);
        free(result);
        return ORC_EINVAL;
    }
    for (size_t b = 0; b < batch; ++b) {
        for (size_t i = 0; i < k; ++i) xh[b * k + i] = x[b * k + i] * orc_half_to_float(suh[i]);
        for (size_t blk = 0; blk < k; blk += 128) h128_block(xh + b * k + blk);
    }
    uint16_t tile[256];
    for (size_t rk = 0; rk < k / 16; ++rk)
        for (size_t cn = 0; cn < n / 16; ++cn) {
            decode_tile_unchecked(packed + (rk * (n / 16) + cn) * 16u * bits, bits, table, tile, 16);
            for (size_t row = 0; row < 16; ++row)
                for (size_t col = 0; col < 16; ++col) {
                    const float w = orc_half_to_float(tile[row * 16 + col]);
                    for (size_t b = 0; b < batch; ++b) result[b * n + cn * 16 + col] += xh[b * k + rk * 16 + row] * w;
                }
        }
    for (size_t b = 0; b < batch; ++b) {
        for (size_t blk = 0; blk < n; blk += 128) h128_block(result + b * n + blk);
        for (size_t i = 0; i < n; ++i) y[b * n + i] = result[b * n + i] * orc_half_to_float(svh[i]);
    }
    free(xh);
    free(result);
    return ORC_OK;
}
