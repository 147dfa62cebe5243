// The namespace exl3 codec API of include/exl3_codec.h, served by the GPU
// library, driven the way the reference's own codec test drives its CPU codec
// (tests/test_codec.cpp:14-97): the mul1 closed form over all 65,536 states,
// binary16 round trips and rounding cases, H128 as an involution, the
// all-zero tile for every rate and codebook, and std::invalid_argument for a
// bad rate or column slice.  Two more checks tie the bulk calls together:
// decode_inner of a 2 x 3 tile matrix equals decode_tile of each tile, and
// reconstruct_slice equals the matching columns of reconstruct.
#include "exl3_codec.h"

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

int failures = 0;

void expect(bool ok, const std::string &what) {
    if (!ok) {
        std::printf("FAIL: %s\n", what.c_str());
        ++failures;
    }
}

template <typename F>
bool throws_invalid_argument(F &&f) {
    try {
        f();
    } catch (const std::invalid_argument &) {
        return true;
    }
    return false;
}

uint32_t next(uint32_t &s) {  // xorshift32
    s ^= s << 13;
    s ^= s >> 17;
    s ^= s << 5;
    return s;
}

}  // namespace

int main() {
    using exl3::Codebook;

    // mul1: w = RNE_f16((1774 s - 905216) / 2^18), s the byte sum of state * 0x83dcd12d
    int bad_mul1 = 0;
    for (uint32_t state = 0; state < 65536; ++state) {
        const uint32_t p = state * 0x83dcd12du;
        const int s = (int)(p & 0xff) + (int)((p >> 8) & 0xff) + (int)((p >> 16) & 0xff) + (int)(p >> 24);
        const float w = std::ldexp((float)(1774 * s - 905216), -18);
        if (exl3::decode_codebook((uint16_t)state, Codebook::mul1) != exl3::float_to_half(w)) ++bad_mul1;
    }
    expect(bad_mul1 == 0, "mul1 closed form over all states (" + std::to_string(bad_mul1) + " differ)");

    // binary16 -> binary32 -> binary16 is the identity on every non-NaN, non-Inf pattern
    int bad_trip = 0;
    for (uint32_t h = 0; h < 65536; ++h)
        if ((h & 0x7c00) != 0x7c00 && exl3::float_to_half(exl3::half_to_float((uint16_t)h)) != h) ++bad_trip;
    expect(bad_trip == 0, "fp16 round trip (" + std::to_string(bad_trip) + " differ)");
    expect(exl3::float_to_half(1.0f + 0x1p-11f) == 0x3c00, "tie rounds to the even neighbour 1.0");
    expect(exl3::float_to_half(1.0f + 3 * 0x1p-11f) == 0x3c02, "tie above an odd mantissa rounds up");
    expect(exl3::float_to_half(65520.0f) == 0x7c00, "65520 rounds to +Inf");
    expect(exl3::float_to_half(-0x1p-25f) == 0x8000, "half the smallest subnormal rounds to -0");
    expect(exl3::half_to_float(0x0001) == 0x1p-24f, "smallest subnormal");

    // H128 applied twice is the identity (it is symmetric and orthonormal)
    std::vector<float> v(3 * 128), v0;
    uint32_t seed = 0x78ef12abu;
    for (float &e : v) e = (float)((int)(next(seed) % 2001) - 1000) / 997.0f;
    v0 = v;
    exl3::hadamard128(v.data(), v.size());
    double moved = 0;
    for (size_t i = 0; i < v.size(); ++i) moved += std::fabs(v[i] - v0[i]);
    expect(moved > 1.0, "H128 changes its input");
    exl3::hadamard128(v.data(), v.size());
    float worst = 0;
    for (size_t i = 0; i < v.size(); ++i) worst = std::fmax(worst, std::fabs(v[i] - v0[i]));
    expect(worst < 1e-6f, "H128 is an involution (max error " + std::to_string(worst) + ")");

    // an all-zero tile decodes to the codebook value of state 0 at every position
    std::vector<uint16_t> zero(16 * 8, 0), tile(256);
    for (unsigned bits = 1; bits <= 8; ++bits)
        for (uint32_t cb = 0; cb < 3; ++cb) {
            const Codebook c = static_cast<Codebook>(cb);
            exl3::decode_tile(zero.data(), bits, c, tile.data());
            const uint16_t want = exl3::decode_codebook(0, c);
            bool all = true;
            for (uint16_t t : tile) all &= t == want;
            expect(all, "zero ring, bits " + std::to_string(bits) + " codebook " + std::to_string(cb));
        }

    // decode_inner is decode_tile at every tile position: k = 32, n = 48 at 3 bits
    {
        const size_t k = 32, n = 48;
        const unsigned bits = 3;
        std::vector<uint16_t> packed((k / 16) * (n / 16) * 16 * bits), whole(k * n), one(256);
        for (uint16_t &p : packed) p = (uint16_t)next(seed);
        exl3::decode_inner(packed.data(), k, n, bits, Codebook::mcg, whole.data());
        bool same = true;
        for (size_t rk = 0; rk < k / 16; ++rk)
            for (size_t cn = 0; cn < n / 16; ++cn) {
                exl3::decode_tile(packed.data() + (rk * (n / 16) + cn) * 16 * bits, bits, Codebook::mcg, one.data());
                for (size_t r = 0; r < 16; ++r)
                    for (size_t c = 0; c < 16; ++c) same &= one[r * 16 + c] == whole[(rk * 16 + r) * n + cn * 16 + c];
            }
        expect(same, "decode_inner agrees with decode_tile per tile");
    }

    // reconstruct_slice is the matching column range of reconstruct
    {
        const size_t k = 128, n = 384, first = 128, count = 256;
        const unsigned bits = 4;
        std::vector<uint16_t> packed((k / 16) * (n / 16) * 16 * bits), su(k), sv(n);
        for (uint16_t &p : packed) p = (uint16_t)next(seed);
        for (uint16_t &s : su) s = (next(seed) & 1) ? 0x3c00 : 0xbc00;
        for (uint16_t &s : sv) s = exl3::float_to_half(0.5f + (float)(next(seed) % 1000) / 1000.0f);
        std::vector<uint16_t> full(k * n), part(k * count);
        exl3::reconstruct(packed.data(), su.data(), sv.data(), k, n, bits, Codebook::mul1, full.data());
        exl3::reconstruct_slice(packed.data(), su.data(), sv.data(), k, n, first, count, bits, Codebook::mul1,
                                part.data());
        bool same = true;
        for (size_t r = 0; r < k; ++r)
            for (size_t c = 0; c < count; ++c) same &= part[r * count + c] == full[r * n + first + c];
        expect(same, "reconstruct_slice agrees with reconstruct");
    }

    // invalid arguments throw std::invalid_argument
    expect(throws_invalid_argument([&] { exl3::decode_tile(zero.data(), 0, Codebook::mul1, tile.data()); }),
           "bits 0 rejected");
    expect(throws_invalid_argument([&] { exl3::decode_tile(zero.data(), 9, Codebook::mul1, tile.data()); }),
           "bits 9 rejected");
    expect(throws_invalid_argument(
               [&] { exl3::decode_inner_slice(zero.data(), 16, 16, 16, 16, 4, Codebook::mul1, tile.data()); }),
           "column slice past the end rejected");
    expect(throws_invalid_argument([&] { exl3::hadamard128(v.data(), 100); }), "H128 of a partial block rejected");

    if (failures) {
        std::printf("%d check(s) failed\n", failures);
        return 1;
    }
    std::printf("PASS: mul1 closed form, fp16 round trip and rounding, H128 involution, zero ring, "
                "inner/tile and slice agreement, argument rejection\n");
    return 0;
}
