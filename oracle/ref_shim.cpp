// ref_shim.cpp -- C entry points over the reference codec (src/exl3_codec.cpp),
// compiled together with the reference's own source file where it lies under
// the reference checkout, into oracle/_ref/libexl3ref.so (see oracle/Makefile).
// Test infrastructure only: used to generate tests/golden/ and to pin the
// oracle restatement bit for bit.  Exceptions become return code 1.
#include "exl3_codec.h"

#include <cstddef>
#include <cstdint>
#include <exception>

extern "C" {

float ref_half_to_float(uint16_t v) { return exl3::half_to_float(v); }
uint16_t ref_float_to_half(float v) { return exl3::float_to_half(v); }

int ref_decode_codebook(uint16_t state, unsigned cb, uint16_t *out) {
    try { *out = exl3::decode_codebook(state, static_cast<exl3::Codebook>(cb)); return 0; }
    catch (const std::exception &) { return 1; }
}

int ref_decode_tile(const uint16_t *packed, unsigned bits, unsigned cb, uint16_t *out) {
    try { exl3::decode_tile(packed, bits, static_cast<exl3::Codebook>(cb), out); return 0; }
    catch (const std::exception &) { return 1; }
}

int ref_decode_inner_slice(const uint16_t *packed, size_t k, size_t n, size_t first, size_t count,
                           unsigned bits, unsigned cb, uint16_t *out) {
    try { exl3::decode_inner_slice(packed, k, n, first, count, bits, static_cast<exl3::Codebook>(cb), out); return 0; }
    catch (const std::exception &) { return 1; }
}

int ref_hadamard128(float *values, size_t count) {
    try { exl3::hadamard128(values, count); return 0; }
    catch (const std::exception &) { return 1; }
}

int ref_reconstruct_slice(const uint16_t *packed, const uint16_t *su, const uint16_t *sv, size_t k,
                          size_t n, size_t first, size_t count, unsigned bits, unsigned cb, uint16_t *out) {
    try { exl3::reconstruct_slice(packed, su, sv, k, n, first, count, bits, static_cast<exl3::Codebook>(cb), out); return 0; }
    catch (const std::exception &) { return 1; }
}

}  // extern "C"
