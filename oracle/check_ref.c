/* check_ref.c -- exhaustive comparison of the oracle restatement with the
 * compiled reference codec (oracle/_ref/libexl3ref.so).  Test infrastructure.
 *   - all 2^16 binary16 -> binary32 conversions (bit patterns, NaNs included)
 *   - all 2^32 binary32 -> binary16 conversions
 *   - all 3 x 65536 codebook states
 *   - 2000 random tiles for every bits 1..8 x codebook 0..2
 * Exit status 0 when everything agrees. */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "exl3_oracle.h"

float ref_half_to_float(uint16_t v);
uint16_t ref_float_to_half(float v);
int ref_decode_codebook(uint16_t state, unsigned cb, uint16_t *out);
int ref_decode_tile(const uint16_t *packed, unsigned bits, unsigned cb, uint16_t *out);

static uint64_t splitmix(uint64_t *s)
{
    uint64_t z = (*s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

int main(void)
{
    unsigned long bad = 0;
    for (uint32_t h = 0; h < 65536u; ++h) {
        float a = orc_half_to_float((uint16_t)h), b = ref_half_to_float((uint16_t)h);
        if (memcmp(&a, &b, 4)) ++bad;
    }
    printf("half_to_float: %lu mismatches over 65536\n", bad);
    unsigned long bad2 = 0;
    uint32_t u = 0;
    do {
        float f;
        memcpy(&f, &u, 4);
        if (orc_float_to_half(f) != ref_float_to_half(f)) ++bad2;
    } while (++u != 0);
    printf("float_to_half: %lu mismatches over 2^32\n", bad2);
    unsigned long bad3 = 0;
    for (unsigned cb = 0; cb < 3; ++cb)
        for (uint32_t s = 0; s < 65536u; ++s) {
            uint16_t r;
            if (ref_decode_codebook((uint16_t)s, cb, &r) || r != orc_decode_codebook((uint16_t)s, cb)) ++bad3;
        }
    printf("decode_codebook: %lu mismatches over 3x65536\n", bad3);
    unsigned long bad4 = 0;
    uint64_t seed = 12345;
    uint16_t packed[128], a[256], b[256];
    for (unsigned bits = 1; bits <= 8; ++bits)
        for (unsigned cb = 0; cb < 3; ++cb)
            for (int t = 0; t < 2000; ++t) {
                for (unsigned i = 0; i < 16 * bits; ++i) packed[i] = (uint16_t)splitmix(&seed);
                if (ref_decode_tile(packed, bits, cb, a) || orc_decode_tile(packed, bits, cb, b) ||
                    memcmp(a, b, sizeof a))
                    ++bad4;
            }
    printf("decode_tile: %lu mismatches over 48000 random tiles\n", bad4);
    return (bad || bad2 || bad3 || bad4) ? 1 : 0;
}
