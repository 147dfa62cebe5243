// exl3_model_format.cpp -- the four passes of exl3_model_format.hpp.  Host C++17
// only; the JSON is read by exl3_json.hpp.  Check semantics and messages follow
// the reference reader, src/exl3_model.cpp:22-156.
#include "exl3_model_format.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <fstream>
#include <iterator>
#include <limits>
#include <stdexcept>

#include "exl3_json.hpp"

namespace exl3fmt {
namespace {

using exl3json::Value;

[[noreturn]] void reject(const std::string &why) { throw std::runtime_error(why); }

// A dimension or offset: a JSON integer, positive (or zero where allowed).
size_t json_count(const Value &v, bool zero_ok) {
    if (!v.is_int()) reject("Expected an integer dimension or offset");
    if (v.integer < 0 || (v.integer == 0 && !zero_ok)) reject("Invalid dimension or offset");
    return static_cast<size_t>(v.integer);
}

// The values a JSON container yields when iterated (an array's items, an
// object's member values); a null yields none and any other value itself.
// A safetensors "shape" is an array; the other forms keep the reference's
// reading of malformed headers (its JSON library iterates them that way).
template <typename F>
void for_each_value(const Value &v, F &&f) {
    switch (v.kind) {
    case Value::Null: return;
    case Value::Array:
        for (const Value &item : v.items) f(item);
        return;
    case Value::Object:
        for (const auto &member : v.members) f(member.second);
        return;
    default: f(v);
    }
}

const std::string &json_text(const Value &v) {
    if (!v.is_string()) reject("Expected a JSON string");
    return v.text;
}

struct DTypeName {
    const char *name;
    DType type;
};
constexpr DTypeName kDTypes[] = {
    {"F16", DType::F16}, {"BF16", DType::BF16}, {"I16", DType::I16}, {"F32", DType::F32}, {"I32", DType::I32}};

DType parse_dtype(const Value &v) {
    const std::string &s = json_text(v);
    for (const DTypeName &d : kDTypes)
        if (s == d.name) return d.type;
    reject("Unsupported model dtype");
}

// One header member -> entry; its span must lie inside the payload and hold
// exactly the shape's elements.
TensorEntry parse_entry(const std::string &name, const Value &info, size_t payload_bytes) {
    TensorEntry e;
    e.name = name;
    e.dtype = parse_dtype(info.at("dtype"));
    size_t elements = 1;
    for_each_value(info.at("shape"), [&](const Value &d) {
        const size_t dim = json_count(d, false);
        if (elements > std::numeric_limits<size_t>::max() / dim) reject("Tensor shape overflow");
        elements *= dim;
        e.dims.push_back(dim);
    });
    const Value &pair = info.at("data_offsets");
    if (!pair.is_array() || pair.items.size() != 2) reject("Invalid tensor offset pair");
    const size_t first = json_count(pair.items[0], true), last = json_count(pair.items[1], true);
    const size_t width = dtype_bytes(e.dtype);
    const bool span_ok = first <= last && last <= payload_bytes &&
                         elements <= std::numeric_limits<size_t>::max() / width && last - first == elements * width;
    if (!span_ok) reject("Invalid tensor data span");
    e.offset = first;
    e.bytes = last - first;
    return e;
}

// The spans, ordered by offset, must start at 0, follow each other without gap
// or overlap and end at the payload's end.
void check_coverage(const std::vector<TensorEntry> &entries, size_t payload_bytes) {
    std::vector<std::pair<size_t, size_t>> spans;  // (offset, end)
    spans.reserve(entries.size());
    for (const TensorEntry &e : entries) spans.emplace_back(e.offset, e.offset + e.bytes);
    std::sort(spans.begin(), spans.end());
    if (!spans.empty() && spans.front().first != 0) reject("Overlapping or missing tensor data");
    const auto seam = std::adjacent_find(spans.begin(), spans.end(),
                                         [](const auto &a, const auto &b) { return a.second != b.first; });
    if (seam != spans.end()) reject("Overlapping or missing tensor data");
    const size_t covered = spans.empty() ? 0 : spans.back().second;
    if (covered != payload_bytes) reject("Unaccounted model payload");
}

uint32_t read_u32_le(const uint8_t *p) {
    return uint32_t(p[0]) | uint32_t(p[1]) << 8 | uint32_t(p[2]) << 16 | uint32_t(p[3]) << 24;
}

std::string slurp(const std::string &path) {
    std::ifstream in(path, std::ios::binary);
    if (!in) reject("Cannot open deployment manifest");
    return std::string(std::istreambuf_iterator<char>(in), std::istreambuf_iterator<char>());
}

bool ends_with(const std::string &s, const std::string &tail) {
    return s.size() > tail.size() && s.compare(s.size() - tail.size(), tail.size(), tail) == 0;
}

}  // namespace

size_t dtype_bytes(DType t) { return (t == DType::F32 || t == DType::I32) ? 4 : 2; }

const char *dtype_name(DType t) {
    for (const DTypeName &d : kDTypes)
        if (d.type == t) return d.name;
    return "?";
}

bool TensorEntry::is(DType t, std::initializer_list<size_t> shape) const {
    return dtype == t && dims.size() == shape.size() && std::equal(dims.begin(), dims.end(), shape.begin());
}

const TensorEntry *TensorIndex::find(const std::string &name) const {
    const auto it = std::lower_bound(entries.begin(), entries.end(), name,
                                     [](const TensorEntry &e, const std::string &key) { return e.name < key; });
    return it != entries.end() && it->name == name ? &*it : nullptr;
}

const TensorEntry &TensorIndex::get(const std::string &name) const {
    const TensorEntry *e = find(name);
    if (!e) reject("Missing model tensor: " + name);
    return *e;
}

WeightFile WeightFile::map(const std::string &path) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) reject("Cannot open model weights");
    // the mapping keeps the file; the descriptor is closed on every path
    struct Descriptor {
        int fd;
        ~Descriptor() { ::close(fd); }
    } guard{fd};
    struct stat st {};
    if (::fstat(fd, &st) != 0 || st.st_size < 8) reject("Invalid weight file size");
    const size_t bytes = static_cast<size_t>(st.st_size);
    void *base = ::mmap(nullptr, bytes, PROT_READ, MAP_PRIVATE, fd, 0);
    if (base == MAP_FAILED) reject("Cannot map model weights");
    WeightFile wf;
    wf.size_ = bytes;
    wf.base_ = std::shared_ptr<const uint8_t>(static_cast<const uint8_t *>(base),
                                              [bytes](const uint8_t *p) { ::munmap(const_cast<uint8_t *>(p), bytes); });
    return wf;
}

TensorIndex index_tensors(const uint8_t *file, size_t file_bytes) {
    // u64 little-endian header length, then the JSON header, then the payload
    uint64_t header_bytes = 0;
    for (int i = 7; i >= 0; --i) header_bytes = header_bytes << 8 | file[i];
    if (header_bytes > (64u << 20) || header_bytes > file_bytes - 8) reject("Invalid safetensors header length");
    TensorIndex ix;
    ix.payload_begin = 8 + static_cast<size_t>(header_bytes);
    ix.payload_bytes = file_bytes - ix.payload_begin;
    const char *text = reinterpret_cast<const char *>(file + 8);
    const Value header = exl3json::parse(text, text + header_bytes);
    if (!header.is_object()) reject("Invalid safetensors header");
    for (const auto &member : header.members) {
        if (member.first == "__metadata__") continue;
        ix.entries.push_back(parse_entry(member.first, member.second, ix.payload_bytes));
    }
    std::sort(ix.entries.begin(), ix.entries.end(),
              [](const TensorEntry &a, const TensorEntry &b) { return a.name < b.name; });
    check_coverage(ix.entries, ix.payload_bytes);
    return ix;
}

Manifest read_manifest(const std::string &json) {
    const Value doc = exl3json::parse(json.data(), json.data() + json.size());
    if (!doc.at("format").equals("hexagon-exl3") || !doc.at("version").equals(1) || !doc.at("kv_cache").equals("f16"))
        reject("Unsupported deployment manifest");
    const Value &alias = doc.at("input_embedding");
    if (!alias.at("type").equals("tied_linear") || !alias.at("basis").equals("original") ||
        !alias.at("token_axis").equals(1))
        reject("Unsupported embedding alias");
    Manifest m;
    m.hidden = json_count(alias.at("hidden_size"), false);
    m.vocab = json_count(alias.at("vocab_size"), false);
    const bool geometry_ok = m.hidden % 128 == 0 && m.vocab % 128 == 0 && m.hidden <= 16384 && m.vocab <= 1048576;
    if (!geometry_ok) reject("Invalid embedding geometry");
    m.parameters = json_count(doc.at("reference_parameter_count"), false);
    m.payload_bytes = json_count(doc.at("weight_payload_bytes"), false);
    m.head = json_text(alias.at("source"));
    return m;
}

int codebook_of(const TensorIndex &index, const uint8_t *file, const std::string &prefix) {
    const TensorEntry *mul1 = index.find(prefix + ".mul1");
    const TensorEntry *mcg = index.find(prefix + ".mcg");
    if (mul1 && mcg) reject("Ambiguous head codebook");
    const TensorEntry *marker = mul1 ? mul1 : mcg;
    if (!marker) return 0;  // three_inst
    if (marker->dtype != DType::I32 || marker->bytes != 4) reject("Invalid codebook marker");
    const uint32_t multiplier = read_u32_le(file + index.payload_begin + marker->offset);
    if (mul1) {
        if (multiplier != 0x83dcd12du) reject("Unsupported mul1 codebook multiplier");
        return 2;
    }
    if (multiplier != 0xcbac1fedu) reject("Unsupported mcg codebook multiplier");
    return 1;
}

HeadBinding bind_head(const TensorIndex &index, const uint8_t *file, const Manifest &m) {
    if (m.payload_bytes != index.payload_bytes || double(index.payload_bytes) * 8 / double(m.parameters) > 5.0)
        reject("Model payload or budget mismatch");
    const TensorEntry &trellis = index.get(m.head + ".trellis");
    const auto &d = trellis.dims;
    const bool trellis_ok = trellis.dtype == DType::I16 && d.size() == 3 && d[0] == m.hidden / 16 &&
                            d[1] == m.vocab / 16 && d[2] % 16 == 0 && d[2] >= 16 && d[2] <= 128;
    if (!trellis_ok) reject("Invalid head trellis");
    if (!index.get(m.head + ".suh").is(DType::F16, {m.hidden}) || !index.get(m.head + ".svh").is(DType::F16, {m.vocab}))
        reject("Invalid head scale");
    HeadBinding h;
    h.bits = unsigned(d[2] / 16);
    h.codebook = codebook_of(index, file, m.head);
    return h;
}

std::vector<MatrixEntry> list_matrices(const TensorIndex &index, const uint8_t *file) {
    static const std::string kTrellis = ".trellis";
    std::vector<MatrixEntry> out;
    for (const TensorEntry &t : index.entries) {  // name order
        if (!ends_with(t.name, kTrellis)) continue;
        const auto &d = t.dims;
        if (t.dtype != DType::I16 || d.size() != 3 || d[2] % 16 || d[2] < 16 || d[2] > 128) continue;
        MatrixEntry m;
        m.prefix = t.name.substr(0, t.name.size() - kTrellis.size());
        m.k = d[0] * 16;
        m.n = d[1] * 16;
        const TensorEntry *su = index.find(m.prefix + ".suh"), *sv = index.find(m.prefix + ".svh");
        if (!su || !sv || !su->is(DType::F16, {m.k}) || !sv->is(DType::F16, {m.n})) continue;
        m.bits = unsigned(d[2] / 16);
        m.codebook = codebook_of(index, file, m.prefix);
        out.push_back(std::move(m));
    }
    return out;
}

std::vector<EmbeddingTableEntry> list_embedding_tables(const TensorIndex &index) {
    static const std::string kTrellis = ".trellis";
    std::vector<EmbeddingTableEntry> out;
    for (const TensorEntry &t : index.entries) {
        if (!ends_with(t.name, kTrellis)) continue;
        const std::string prefix = t.name.substr(0, t.name.size() - kTrellis.size());
        const TensorEntry *signs = index.find(prefix + ".signs");
        if (!signs) continue;  // a matrix trellis
        // [rows, groups * words] I16 codes with [groups, 256] F16 signs
        const bool shape_ok = t.dims.size() == 2 && t.dtype == DType::I16 && signs->dtype == DType::F16 &&
                              signs->dims.size() == 2 && signs->dims[1] == 256;
        if (!shape_ok) reject("Invalid EXL3 embedding: " + t.name);
        const size_t groups = signs->dims[0];
        if (groups == 0 || t.dims[1] % groups) reject("Invalid EXL3 embedding groups: " + t.name);
        // each group of a row: one 16-bit header word plus 16 words per bit of rate
        const size_t words = t.dims[1] / groups;
        if ((words - 1) % 16 || (words - 1) / 16 < 1 || (words - 1) / 16 > 8)
            reject("Invalid EXL3 embedding bitrate: " + t.name);
        EmbeddingTableEntry e;
        e.prefix = prefix;
        e.rows = t.dims[0];
        e.groups = groups;
        e.width_padded = groups * 256;
        e.bits = unsigned((words - 1) / 16);
        out.push_back(std::move(e));
    }
    return out;
}

OpenedModel open_model(const std::string &directory) {
    OpenedModel om;
    om.file = WeightFile::map(directory + "/model.safetensors");
    om.index = index_tensors(om.file.bytes(), om.file.size());
    om.manifest = read_manifest(slurp(directory + "/hexagon-exl3.json"));
    om.head = bind_head(om.index, om.file.bytes(), om.manifest);
    return om;
}

}  // namespace exl3fmt
