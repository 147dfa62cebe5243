// exl3::Model (include/exl3_model.h) driven as the reference's reader test
// drives its own (tests/test_model_reader.cpp:23-73): a 128 x 128 4-bit
// all-zero trellis used as the tied embedding with su = sv = 1 and a mul1
// marker.  H128 of a constant column is sqrt(128) at index 0 and zero
// elsewhere, so token 0's row is fp16(128 * code(0)) followed by zeros and
// every other token's row is zero.  Then four malformed variants (parameter
// budget, overlapping spans, a negative dimension, a truncated payload) must be
// rejected.  The directory comes from the command line (a fresh empty one).
#include "exl3_model.h"
#include "exl3_codec.h"

#include <cstdint>
#include <cstdio>
#include <fstream>
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

struct Case {
    long long param_count = 16384;
    long long suh_begin = 8192, suh_end = 8448;
    long long suh_dim = 128;
    size_t payload = 8708;
};

std::string header_json(const Case &c) {
    return std::string("{") +
           "\"lm_head.trellis\":{\"dtype\":\"I16\",\"shape\":[8,8,64],\"data_offsets\":[0,8192]}," +
           "\"lm_head.suh\":{\"dtype\":\"F16\",\"shape\":[" + std::to_string(c.suh_dim) + "],\"data_offsets\":[" +
           std::to_string(c.suh_begin) + "," + std::to_string(c.suh_end) + "]}," +
           "\"lm_head.svh\":{\"dtype\":\"F16\",\"shape\":[128],\"data_offsets\":[8448,8704]}," +
           "\"lm_head.mul1\":{\"dtype\":\"I32\",\"shape\":[],\"data_offsets\":[8704,8708]}}";
}

std::string manifest_json(const Case &c) {
    return std::string("{\"format\":\"hexagon-exl3\",\"version\":1,\"kv_cache\":\"f16\",") +
           "\"reference_parameter_count\":" + std::to_string(c.param_count) + ",\"weight_payload_bytes\":8708," +
           "\"input_embedding\":{\"type\":\"tied_linear\",\"source\":\"lm_head\",\"basis\":\"original\"," +
           "\"token_axis\":1,\"hidden_size\":128,\"vocab_size\":128}}";
}

void write_model(const std::string &dir, const Case &c) {
    std::string text = header_json(c);
    text.append((8 - text.size() % 8) % 8, ' ');
    std::vector<uint8_t> data(8708, 0);
    for (size_t i = 8192; i < 8704; i += 2) data[i + 1] = 0x3c;  // su = sv = 1.0
    const uint32_t marker = 0x83dcd12du;
    for (int i = 0; i < 4; ++i) data[8704 + i] = (uint8_t)(marker >> (8 * i));
    data.resize(c.payload);
    std::ofstream w(dir + "/model.safetensors", std::ios::binary | std::ios::trunc);
    const uint64_t len = text.size();
    for (int i = 0; i < 8; ++i) w.put((char)(len >> (8 * i)));
    w.write(text.data(), (std::streamsize)text.size());
    w.write((const char *)data.data(), (std::streamsize)data.size());
    std::ofstream m(dir + "/hexagon-exl3.json", std::ios::trunc);
    m << manifest_json(c);
}

bool rejected(const std::string &dir, const Case &c) {
    write_model(dir, c);
    try {
        exl3::Model model(dir);
    } catch (const std::exception &) {
        return true;
    }
    return false;
}

}  // namespace

int main(int argc, char **argv) {
    if (argc != 2) {
        std::printf("usage: test_model_api <empty directory>\n");
        return 2;
    }
    const std::string dir = argv[1];
    try {
        write_model(dir, Case{});
        exl3::Model model(dir);
        expect(model.tensor_count() == 4, "four tensors");
        expect(model.payload_bytes() == 8708, "payload bytes");
        expect(model.hidden_size() == 128 && model.vocab_size() == 128, "embedding geometry");
        const std::vector<uint16_t> row0 = model.embedding(0), row1 = model.embedding(1);
        expect(row0.size() == 128 && row1.size() == 128, "row length = hidden size");
        expect(model.embedding(0) == row0, "a cached row is returned unchanged");
        const float code0 = exl3::half_to_float(exl3::decode_codebook(0, exl3::Codebook::mul1));
        expect(row0[0] == exl3::float_to_half(128.0f * code0), "token 0: 128 code(0) at index 0");
        bool rest_zero = true, row1_zero = true;
        for (size_t i = 1; i < row0.size(); ++i) rest_zero &= exl3::half_to_float(row0[i]) == 0.0f;
        for (uint16_t v : row1) row1_zero &= exl3::half_to_float(v) == 0.0f;
        expect(rest_zero, "token 0: zeros after index 0");
        expect(row1_zero, "token 1: all zeros");
        bool out_of_range = false;
        try {
            model.embedding(128);
        } catch (const std::invalid_argument &) {
            out_of_range = true;
        }
        expect(out_of_range, "token 128 rejected with std::invalid_argument");
        const auto mats = model.matrices();
        expect(mats.size() == 1 && mats[0].prefix == "lm_head" && mats[0].bits == 4 &&
                   mats[0].codebook == exl3::Codebook::mul1 && mats[0].k == 128 && mats[0].n == 128,
               "matrix inventory");
        expect(!mats.empty() && model.record_bytes(mats[0]) == 8704, "record bytes of one 4-bit record");
    } catch (const std::exception &e) {
        std::printf("FAIL: the reference case threw: %s\n", e.what());
        ++failures;
    }
    Case c;
    c.param_count = 1;
    expect(rejected(dir, c), "parameter budget exceeded");
    c = Case{};
    c.suh_begin = 8190;
    c.suh_end = 8446;
    expect(rejected(dir, c), "overlapping tensor spans");
    c = Case{};
    c.suh_dim = -128;
    expect(rejected(dir, c), "negative dimension");
    c = Case{};
    c.payload = 8707;
    expect(rejected(dir, c), "truncated payload");
    std::remove((dir + "/model.safetensors").c_str());
    std::remove((dir + "/hexagon-exl3.json").c_str());
    if (failures) {
        std::printf("%d check(s) failed\n", failures);
        return 1;
    }
    std::printf("PASS: tied embedding known answer, row cache, token bound, inventory, budget, overlapping "
                "spans, negative dimension, truncation\n");
    return 0;
}
