/*
 * exl3-block.h -- the 128x128 EXL3 group-record layout.
 *
 * Same names, type ids and byte layout as the reference's include/exl3-block.h
 * (lines 5-14 and 34-39), so records written for the reference's ggml types
 * 43/44/45 are consumed unchanged by the HIP path.
 *
 * A record covers 128 input rows (k) x 128 output columns (n):
 *   [ 64 trellis tiles of 32*bits bytes, tile (r, c) at byte (8 r + c) * 32 * bits ]
 *   [ su[128] fp16 : input scales of this record's 128 rows    ]
 *   [ sv[128] fp16 : output scales of this record's 128 columns ]
 * Record (nb, kb) of a k x n matrix starts at byte (nb * (k / 128) + kb) * exl3_group_bytes(bits),
 * i.e. records are column-group-major, so a 128-column group is one contiguous run.
 *
 * The Hexagon VTCM scratch planners of the reference header (exl3_thread_bytes,
 * exl3_row_chunk, exl3_hmx_*) size DSP scratch memory and have no meaning on the GPU;
 * they are not provided.
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#define EXL3_TYPE_4 43
#define EXL3_TYPE_6 44
#define EXL3_TYPE_8 45
#define EXL3_GROUP_DIM 128

/* ggml type id -> bits per weight (0 if not an EXL3 type); include/exl3-block.h:11-13 */
static inline unsigned exl3_type_bits(unsigned type) {
    switch (type) {
    case EXL3_TYPE_4: return 4;
    case EXL3_TYPE_6: return 6;
    case EXL3_TYPE_8: return 8;
    default: return 0;
    }
}

/* bytes of one 128x128 record; include/exl3-block.h:14 */
static inline size_t exl3_group_bytes(unsigned bits) { return (size_t) 2048 * bits + 512; }

/* the record's su / sv vectors; include/exl3-block.h:34-39 */
static inline const uint16_t * exl3_group_su(const void * group, unsigned bits) {
    return (const uint16_t *) ((const unsigned char *) group + (size_t) 2048 * bits);
}
static inline const uint16_t * exl3_group_sv(const void * group, unsigned bits) {
    return (const uint16_t *) ((const unsigned char *) group + (size_t) 2048 * bits + 256);
}
