/*
 * exl3_codec.h -- EXL3 codec API, same namespace, names, argument meaning and
 * exception behaviour as the reference's include/exl3_codec.h:8-29.
 *
 * In this library the bulk operations (decode_tile, decode_inner(_slice),
 * hadamard128, reconstruct(_slice)) run on the GPU through the C-ABI of
 * exl3_hip.h: host buffers in, host buffers out, one synchronous call on the
 * current HIP device.  Invalid arguments throw std::invalid_argument as in the
 * reference; a HIP failure throws std::runtime_error.
 */
#pragma once

#include <cstddef>
#include <cstdint>

namespace exl3 {

enum class Codebook : uint32_t { three_inst = 0, mcg = 1, mul1 = 2 };

// IEEE binary16 <-> binary32 (round half to even).  src/exl3_codec.cpp:21-66
float half_to_float(uint16_t value);
uint16_t float_to_half(float value);
// One trellis state -> fp16 bits.  src/exl3_codec.cpp:68-86
uint16_t decode_codebook(uint16_t state, Codebook codebook);

// Packed tiles use upstream tensor-core lane order and little-endian uint16 storage.
// src/exl3_codec.cpp:92-145
void decode_tile(const uint16_t * packed, unsigned bits, Codebook codebook, uint16_t * row_major);
void decode_inner(const uint16_t * packed, size_t k, size_t n, unsigned bits, Codebook codebook,
                  uint16_t * output);
void decode_inner_slice(const uint16_t * packed, size_t k, size_t n, size_t first_column,
                        size_t column_count, unsigned bits, Codebook codebook, uint16_t * output);

// In-place orthonormal H128 on each consecutive group of 128 values.  src/exl3_codec.cpp:147-167
void hadamard128(float * values, size_t count);

// Original-basis matrix: diag(suh) H128 W_hat H128 diag(svh), laid out as [k,n].
// src/exl3_codec.cpp:169-204
void reconstruct(const uint16_t * packed, const uint16_t * suh, const uint16_t * svh,
                 size_t k, size_t n, unsigned bits, Codebook codebook, uint16_t * output);
void reconstruct_slice(const uint16_t * packed, const uint16_t * suh, const uint16_t * svh,
                       size_t k, size_t n, size_t first_column, size_t column_count,
                       unsigned bits, Codebook codebook, uint16_t * output);

} // namespace exl3
