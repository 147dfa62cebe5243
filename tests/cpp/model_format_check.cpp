// Host-only driver for the model reader's format passes
// (xiaomi-hexagon-exl3_amd/csrc/exl3_model_format.cpp) and the JSON reader
// (csrc/exl3_json.hpp), built by tests/test_model_sanitized.py with
// AddressSanitizer and UndefinedBehaviorSanitizer.
//
//   model_format_check DIR...         one line per directory:
//                                     "OPEN <dir> <tensors> <payload> <bits> <codebook> <matrices>"
//                                     or "REJECT <dir>: <reason>"
//   model_format_check --json-fuzz SEED COUNT FILE
//                                     COUNT mutations of FILE's text (truncation,
//                                     byte changes, insertions, deletions) through
//                                     the JSON reader; prints "FUZZ <parsed> <rejected>"
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iterator>
#include <stdexcept>
#include <string>

#include "exl3_json.hpp"
#include "exl3_model_format.hpp"

namespace {

uint64_t splitmix(uint64_t &s) {
    uint64_t z = (s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

int json_fuzz(uint64_t seed, long count, const char *path) {
    std::ifstream in(path, std::ios::binary);
    const std::string base((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
    static const char alphabet[] = "{}[]:,\"\\-+.eE0123456789 tfnulr\x01\xff";
    long parsed = 0, rejected = 0;
    for (long i = 0; i < count; ++i) {
        std::string t = base;
        const int edits = 1 + int(splitmix(seed) % 4);
        for (int e = 0; e < edits && !t.empty(); ++e) {
            const size_t at = splitmix(seed) % t.size();
            const char c = alphabet[splitmix(seed) % (sizeof(alphabet) - 1)];
            switch (splitmix(seed) % 4) {
            case 0: t.resize(at); break;
            case 1: t[at] = c; break;
            case 2: t.insert(t.begin() + long(at), c); break;
            default: t.erase(at, 1 + splitmix(seed) % 8); break;
            }
        }
        try {
            // an exact-size heap copy, so a read past the end is an ASan report
            char *buf = new char[t.size() ? t.size() : 1];
            std::memcpy(buf, t.data(), t.size());
            try {
                (void)exl3json::parse(buf, buf + t.size());
                ++parsed;
            } catch (const std::runtime_error &) {
                ++rejected;
            }
            delete[] buf;
        } catch (const std::exception &ex) {
            std::printf("UNEXPECTED %s\n", ex.what());
            return 1;
        }
    }
    std::printf("FUZZ %ld %ld\n", parsed, rejected);
    return 0;
}

}  // namespace

int main(int argc, char **argv) {
    if (argc >= 5 && std::strcmp(argv[1], "--json-fuzz") == 0)
        return json_fuzz(std::strtoull(argv[2], nullptr, 10), std::strtol(argv[3], nullptr, 10), argv[4]);
    for (int i = 1; i < argc; ++i) {
        try {
            const exl3fmt::OpenedModel om = exl3fmt::open_model(argv[i]);
            const auto mats = exl3fmt::list_matrices(om.index, om.file.bytes());
            std::printf("OPEN %s %zu %zu %u %d %zu\n", argv[i], om.index.entries.size(), om.index.payload_bytes,
                        om.head.bits, om.head.codebook, mats.size());
        } catch (const std::exception &e) {
            std::printf("REJECT %s: %s\n", argv[i], e.what());
        }
    }
    return 0;
}
