/* CPU checks of include/exl3-block.h: the record helpers and the Hexagon VTCM
 * planners the header keeps for source compatibility.  Plain C11, no GPU.
 *
 * Known answers are worked out by hand from the planners' definitions
 * (include/exl3-block.h:15-33 of the reference); the invariants are the
 * properties the reference's codec test requires of every plan
 * (tests/test_codec.cpp:33-57): at most 32 rows, the plan fits the VTCM budget,
 * 2 KiB alignment of the HMX regions, and the HMX output tile behind the HVX
 * scratch of each worker. */
#include <stdio.h>
#include <stdlib.h>

#include "exl3-block.h"

static int failures = 0;
#define CHECK(cond, msg)                                              \
    do {                                                              \
        if (!(cond)) {                                                \
            fprintf(stderr, "FAIL %s (line %d)\n", (msg), __LINE__);  \
            ++failures;                                               \
        }                                                             \
    } while (0)

int main(void) {
    /* type ids and record geometry */
    CHECK(exl3_type_bits(EXL3_TYPE_4) == 4 && exl3_type_bits(EXL3_TYPE_6) == 6 && exl3_type_bits(EXL3_TYPE_8) == 8,
          "type ids 43/44/45");
    CHECK(exl3_type_bits(0) == 0 && exl3_type_bits(42) == 0 && exl3_type_bits(46) == 0, "other types");
    CHECK(exl3_group_bytes(4) == 8704 && exl3_group_bytes(6) == 12800 && exl3_group_bytes(8) == 16896,
          "record bytes 68/100/132 per 128-element row");
    {
        unsigned char rec[16896];
        CHECK((const unsigned char *) exl3_group_su(rec, 4) == rec + 8192, "su offset");
        CHECK((const unsigned char *) exl3_group_sv(rec, 4) == rec + 8448, "sv offset");
        CHECK((const unsigned char *) exl3_group_sv(rec, 8) == rec + 16640, "sv offset at 8 bits");
    }
    CHECK(EXL3_GROUP_DIM == 128 && EXL3_DECODE_PAD_BYTES == 128, "constants");

    /* hand-computed plans: thread bytes at 4 bits and no rows =
     * 32768 + 128 + 0 + 8704 + 640 */
    CHECK(exl3_thread_bytes(4, 0) == 42240, "HVX worker scratch, 4 bits");
    CHECK(exl3_thread_bytes(8, 32) == 32768 + 128 + 32 * 512 + 16896 + 640, "HVX worker scratch, 8 bits, 32 rows");
    /* 4 workers, k = 2048, 256 KiB: (262144 - 4 * 42240) / (8192 + 4 * 512) = 93184 / 10240 -> 9 */
    CHECK(exl3_row_chunk(4, 2048, 4, 262144) == 9, "row chunk 9");
    /* the FFN case of the reference test: 8 MiB holds more than 32 rows */
    CHECK(exl3_row_chunk(4, 6144, 4, 8 * 1024 * 1024) == 32, "FFN row chunk capacity");
    CHECK(exl3_row_chunk(4, 2048, 0, 8 * 1024 * 1024) == 0, "no workers");
    CHECK(exl3_row_chunk(4, 0, 4, 8 * 1024 * 1024) == 0, "no input dimension");
    CHECK(exl3_row_chunk(4, 2048, 4, 4 * 42240) == 0, "budget equal to the fixed scratch");
    CHECK(exl3_hmx_extra(2048, 4) == 2048 * 64 + 256 + 4096 + 4 * 10240, "HMX extra");
    CHECK(exl3_hmx_activation_offset(2048, 3) == 24576, "activation offset, already aligned");
    CHECK(exl3_hmx_activation_offset(100, 3) == 2048, "activation offset rounds up to 2 KiB");
    CHECK(exl3_hmx_thread_bytes(4, 0) == 43008 + 8192, "HMX worker bytes (42240 -> 43008)");
    CHECK(exl3_hmx_prefix_bytes(100, 3) == ((2048 + 6400 + 256 + 2047) & ~(size_t) 2047), "HMX prefix");

    /* invariants over the reference test's grid */
    const unsigned rates[3] = {4, 6, 8};
    const size_t ks[4] = {128, 2048, 6144, 65536};
    const size_t budgets[4] = {131072, 262144, 4194304, 8388608};
    for (int b = 0; b < 3; ++b)
        for (int ki = 0; ki < 4; ++ki)
            for (unsigned threads = 1; threads <= 4; ++threads)
                for (int bi = 0; bi < 4; ++bi) {
                    const unsigned bits = rates[b];
                    const size_t k = ks[ki], budget = budgets[bi];
                    const size_t chunk = exl3_row_chunk(bits, k, threads, budget);
                    CHECK(chunk <= 32, "row chunk bound");
                    if (chunk) {
                        CHECK(chunk * k * 4 + threads * exl3_thread_bytes(bits, chunk) <= budget, "plan fits VTCM");
                        /* maximal: one more row would not fit (or the cap applies) */
                        CHECK(chunk == 32 || (chunk + 1) * (k * 4 + threads * 512) > budget - threads * exl3_thread_bytes(bits, 0),
                              "row chunk is the largest that fits");
                    }
                    const size_t extra = exl3_hmx_extra(k, threads);
                    if (extra >= budget) continue;
                    const size_t hmx_rows = exl3_row_chunk(bits, k, threads, budget - extra);
                    if (!hmx_rows) continue;
                    const size_t prefix = exl3_hmx_prefix_bytes(k, hmx_rows);
                    const size_t per_thread = exl3_hmx_thread_bytes(bits, hmx_rows);
                    CHECK(prefix + threads * per_thread <= budget, "HMX scratch fits VTCM");
                    CHECK(prefix % 2048 == 0 && per_thread % 2048 == 0, "HMX output alignment");
                    CHECK(exl3_hmx_activation_offset(k, hmx_rows) % 2048 == 0, "HMX activation alignment");
                    CHECK(per_thread - 8192 >= exl3_thread_bytes(bits, hmx_rows), "HMX output behind decode scratch");
                }
    if (failures) {
        fprintf(stderr, "%d failures\n", failures);
        return 1;
    }
    printf("PASS: exl3-block.h record helpers and VTCM planners\n");
    return 0;
}
