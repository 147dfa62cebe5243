// exl3_codec_api.cpp -- namespace exl3 codec API (include/exl3_codec.h) served by
// the GPU kernels: each bulk call stages host buffers to the current HIP
// device, runs the kernel through the C-ABI and copies the result back.
// Argument checks and exception types follow src/exl3_codec.cpp:12-19,117-135,
// 147-150,177-180.
#include "exl3_codec.h"

#include <hip/hip_runtime.h>

#include <cstring>
#include <limits>
#include <stdexcept>
#include <string>
#include <vector>

#include "exl3_hip.h"

namespace exl3 {
namespace {

void check_rate(unsigned bits, Codebook codebook) {
    if (bits < 1 || bits > 8) throw std::invalid_argument("EXL3 integer bitrate must be in [1,8]");
    if (static_cast<uint32_t>(codebook) > 2) throw std::invalid_argument("Unknown EXL3 codebook");
}

void check_shape(size_t k, size_t n, size_t multiple) {
    if (!k || !n || k % multiple || n % multiple || k > std::numeric_limits<size_t>::max() / n)
        throw std::invalid_argument("Invalid EXL3 matrix dimensions");
}

void check_slice(size_t n, size_t first, size_t count) {
    if (!count || first % 16 || count % 16 || first > n || count > n - first)
        throw std::invalid_argument("Invalid EXL3 column slice");
}

void hip_check(hipError_t e, const char *what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

void status_check(exl3_status s, const char *what) {
    if (s == EXL3_INVAL_PARAMS) throw std::invalid_argument(std::string(what) + ": invalid parameters");
    if (s != EXL3_OK) throw std::runtime_error(std::string(what) + ": " + exl3_hip_status_string(s));
}

// device buffer owned for the duration of one call
struct DeviceBuffer {
    void *ptr = nullptr;
    explicit DeviceBuffer(size_t bytes) { hip_check(hipMalloc(&ptr, bytes ? bytes : 16), "hipMalloc"); }
    ~DeviceBuffer() { if (ptr) (void)hipFree(ptr); }
    DeviceBuffer(const DeviceBuffer &) = delete;
    DeviceBuffer &operator=(const DeviceBuffer &) = delete;
    template <typename T> T *as() const { return static_cast<T *>(ptr); }
};

void upload(DeviceBuffer &d, const void *src, size_t bytes) { hip_check(hipMemcpy(d.ptr, src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D"); }
void download(void *dst, const DeviceBuffer &d, size_t bytes) { hip_check(hipMemcpy(dst, d.ptr, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H"); }

}  // namespace

// binary16 -> binary32, exact (src/exl3_codec.cpp:21-38)
float half_to_float(uint16_t value) {
    const uint32_t sign = uint32_t(value & 0x8000u) << 16;
    const uint32_t field = (value >> 10) & 0x1fu, frac = value & 0x3ffu;
    uint32_t word;
    if (field == 0) {
        if (!frac) {
            word = sign;
        } else {  // subnormal: normalise the fraction
            int e = -1;
            uint32_t f = frac;
            do { f <<= 1; ++e; } while (!(f & 0x400u));
            word = sign | uint32_t(127 - 15 - e) << 23 | (f & 0x3ffu) << 13;
        }
    } else if (field == 0x1fu) {
        word = sign | 0x7f800000u | frac << 13;
    } else {
        word = sign | (field + 112u) << 23 | frac << 13;
    }
    float out;
    std::memcpy(&out, &word, sizeof out);
    return out;
}

// binary32 -> binary16, round half to even; NaN -> 0x7e00 (src/exl3_codec.cpp:40-66)
uint16_t float_to_half(float value) {
    uint32_t u;
    std::memcpy(&u, &value, sizeof u);
    const uint16_t sign = uint16_t((u >> 16) & 0x8000u);
    const uint32_t e = (u >> 23) & 0xffu, m = u & 0x7fffffu;
    if (e == 0xffu) return uint16_t(sign | (m ? 0x7e00u : 0x7c00u));
    if (e > 142u) return uint16_t(sign | 0x7c00u);
    if (e < 102u) return sign;
    const bool sub = e < 113u;
    const uint32_t mant = sub ? (m | 0x800000u) : m;
    const unsigned sh = sub ? 126u - e : 13u;
    uint32_t q = mant >> sh;
    const uint32_t rem = mant & ((1u << sh) - 1u), half = 1u << (sh - 1u);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return uint16_t(sign | (sub ? q : ((e - 112u) << 10) + q));
}

uint16_t decode_codebook(uint16_t state, Codebook codebook) {
    if (static_cast<uint32_t>(codebook) > 2) throw std::invalid_argument("Unknown EXL3 codebook");
    DeviceBuffer d(4);
    upload(d, &state, 2);
    status_check(exl3_hip_codebook(d.as<uint16_t>(), 1, static_cast<unsigned>(codebook), d.as<uint16_t>() + 1, nullptr),
                 "decode_codebook");
    uint16_t out[2];
    download(out, d, 4);
    return out[1];
}

void decode_inner_slice(const uint16_t *packed, size_t k, size_t n, size_t first_column, size_t column_count,
                        unsigned bits, Codebook codebook, uint16_t *output) {
    check_rate(bits, codebook);
    check_shape(k, n, 16);
    check_slice(n, first_column, column_count);
    const size_t in_bytes = k * n * bits / 8, out_bytes = k * column_count * 2;
    DeviceBuffer din(in_bytes), dout(out_bytes);
    upload(din, packed, in_bytes);
    status_check(exl3_hip_decode(din.ptr, EXL3_LAYOUT_UPSTREAM_TILES, bits, static_cast<unsigned>(codebook), k, n,
                                 first_column, column_count, dout.as<uint16_t>(), nullptr),
                 "decode_inner_slice");
    download(output, dout, out_bytes);
}

void decode_inner(const uint16_t *packed, size_t k, size_t n, unsigned bits, Codebook codebook, uint16_t *output) {
    decode_inner_slice(packed, k, n, 0, n, bits, codebook, output);
}

void decode_tile(const uint16_t *packed, unsigned bits, Codebook codebook, uint16_t *row_major) {
    check_rate(bits, codebook);
    decode_inner_slice(packed, 16, 16, 0, 16, bits, codebook, row_major);
}

void hadamard128(float *values, size_t count) {
    if (count % 128) throw std::invalid_argument("H128 length must be a multiple of 128");
    if (!count) return;
    DeviceBuffer d(count * 4);
    upload(d, values, count * 4);
    status_check(exl3_hip_hadamard128(d.as<float>(), count, nullptr), "hadamard128");
    download(values, d, count * 4);
}

void reconstruct_slice(const uint16_t *packed, const uint16_t *suh, const uint16_t *svh, size_t k, size_t n,
                       size_t first_column, size_t column_count, unsigned bits, Codebook codebook, uint16_t *output) {
    check_shape(k, n, 128);
    if (first_column % 128 || column_count % 128) throw std::invalid_argument("H128 slices must align to 128 columns");
    check_rate(bits, codebook);
    check_slice(n, first_column, column_count);
    const size_t in_bytes = k * n * bits / 8, out_bytes = k * column_count * 2;
    DeviceBuffer din(in_bytes), dsu(k * 2), dsv(n * 2), dout(out_bytes);
    upload(din, packed, in_bytes);
    upload(dsu, suh, k * 2);
    upload(dsv, svh, n * 2);
    status_check(exl3_hip_reconstruct(din.ptr, EXL3_LAYOUT_UPSTREAM_TILES, dsu.as<uint16_t>(), dsv.as<uint16_t>(), bits,
                                      static_cast<unsigned>(codebook), k, n, first_column, column_count,
                                      dout.as<uint16_t>(), nullptr),
                 "reconstruct_slice");
    download(output, dout, out_bytes);
}

void reconstruct(const uint16_t *packed, const uint16_t *suh, const uint16_t *svh, size_t k, size_t n, unsigned bits,
                 Codebook codebook, uint16_t *output) {
    reconstruct_slice(packed, suh, svh, k, n, 0, n, bits, codebook, output);
}

}  // namespace exl3
