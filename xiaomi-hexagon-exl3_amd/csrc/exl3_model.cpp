// exl3_model.cpp -- exl3::Model (include/exl3_model.h): the deployment-model
// reader of src/exl3_model.cpp:22-187 with the same checks, in the same order,
// and the same exception types; the JSON is read by exl3_json.hpp.  The
// embedding's reconstruct and the record packing run on the GPU through the
// C-ABI.  Also the C wrappers exl3_hip_model_* of include/exl3_hip.h.
#include "exl3_model.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <fstream>
#include <iterator>
#include <limits>
#include <list>
#include <map>
#include <mutex>
#include <sstream>
#include <stdexcept>
#include <utility>

#include "exl3_hip.h"
#include "exl3_json.hpp"

namespace exl3 {
namespace {

using exl3json::Value;

// read-only private mapping of the weights (src/exl3_model.cpp:22-42)
struct Mapping {
    int fd = -1;
    size_t size = 0;
    const uint8_t *data = nullptr;
    explicit Mapping(const std::string &path) {
        fd = open(path.c_str(), O_RDONLY);
        if (fd < 0) throw std::runtime_error("Cannot open model weights");
        struct stat st {};
        if (fstat(fd, &st) || st.st_size < 8) {
            close(fd);
            fd = -1;
            throw std::runtime_error("Invalid weight file size");
        }
        size = (size_t)st.st_size;
        void *m = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            close(fd);
            fd = -1;
            throw std::runtime_error("Cannot map model weights");
        }
        data = static_cast<const uint8_t *>(m);
    }
    ~Mapping() {
        if (data) munmap(const_cast<uint8_t *>(data), size);
        if (fd >= 0) close(fd);
    }
    Mapping(const Mapping &) = delete;
    Mapping &operator=(const Mapping &) = delete;
};

// src/exl3_model.cpp:44-49
size_t positive_integer(const Value &v, bool zero_allowed = false) {
    if (!v.is_int()) throw std::runtime_error("Expected an integer dimension or offset");
    if (v.integer < 0 || (!v.integer && !zero_allowed)) throw std::runtime_error("Invalid dimension or offset");
    return (size_t)v.integer;
}

// the elements a range-for visits over a JSON value: an array's items, an
// object's values, nothing for null, the value itself otherwise
std::vector<const Value *> elements_of(const Value &v) {
    std::vector<const Value *> out;
    if (v.kind == Value::Array) {
        for (const auto &x : v.items) out.push_back(&x);
    } else if (v.kind == Value::Object) {
        for (const auto &m : v.members) out.push_back(&m.second);
    } else if (v.kind != Value::Null) {
        out.push_back(&v);
    }
    return out;
}

const std::string &string_of(const Value &v) {
    if (!v.is_string()) throw std::runtime_error("Expected a JSON string");
    return v.text;
}

struct Tensor {
    std::string dtype;
    std::vector<size_t> shape;
    const uint8_t *data = nullptr;
    size_t size = 0;
    const uint16_t *half_data() const {
        if (reinterpret_cast<uintptr_t>(data) % 2) throw std::runtime_error("Unaligned half tensor");
        return reinterpret_cast<const uint16_t *>(data);
    }
};

void hip_check(hipError_t e, const char *what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// device buffer owned by the model or by one call
struct DeviceBuffer {
    void *ptr = nullptr;
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t bytes) { hip_check(hipMalloc(&ptr, bytes ? bytes : 16), "hipMalloc"); }
    ~DeviceBuffer() {
        if (ptr) (void)hipFree(ptr);
    }
    DeviceBuffer(const DeviceBuffer &) = delete;
    DeviceBuffer &operator=(const DeviceBuffer &) = delete;
};

// restores the caller's current device on scope exit
struct DeviceScope {
    int saved = -1;
    explicit DeviceScope(int dev) {
        if (hipGetDevice(&saved) != hipSuccess) saved = -1;
        if (dev >= 0 && dev != saved) hip_check(hipSetDevice(dev), "hipSetDevice");
    }
    ~DeviceScope() {
        if (saved >= 0) (void)hipSetDevice(saved);
    }
};

}  // namespace

struct Model::Impl {
    Mapping weights;
    std::map<std::string, Tensor> tensors;
    size_t payload = 0, k = 0, n = 0, parameters = 0;
    unsigned head_bits = 0;
    Codebook head_codebook = Codebook::three_inst;
    std::string head_prefix;
    mutable std::mutex cache_mutex;
    mutable std::list<std::pair<size_t, std::shared_ptr<std::vector<uint16_t>>>> cache;
    // the head on the device, uploaded by the first embedding() call
    mutable int head_device = -1;
    mutable std::unique_ptr<DeviceBuffer> d_trellis, d_su, d_sv, d_block;

    const Tensor &tensor(const std::string &key) const {
        auto found = tensors.find(key);
        if (found == tensors.end()) throw std::runtime_error("Missing model tensor: " + key);
        return found->second;
    }

    // the codebook a matrix's markers name (src/exl3_model.cpp:140-156)
    Codebook codebook_of(const std::string &prefix) const {
        auto marker = tensors.find(prefix + ".mul1");
        if (marker != tensors.end() && tensors.count(prefix + ".mcg")) throw std::runtime_error("Ambiguous head codebook");
        uint32_t value;
        if (marker != tensors.end()) {
            if (marker->second.dtype != "I32" || marker->second.size != 4) throw std::runtime_error("Invalid codebook marker");
            std::memcpy(&value, marker->second.data, 4);
            if (value != 0x83dcd12du) throw std::runtime_error("Unsupported mul1 codebook multiplier");
            return Codebook::mul1;
        }
        if (tensors.count(prefix + ".mcg")) {
            const Tensor &mcg = tensor(prefix + ".mcg");
            if (mcg.dtype != "I32" || mcg.size != 4) throw std::runtime_error("Invalid codebook marker");
            std::memcpy(&value, mcg.data, 4);
            if (value != 0xcbac1fedu) throw std::runtime_error("Unsupported mcg codebook multiplier");
            return Codebook::mcg;
        }
        return Codebook::three_inst;
    }

    explicit Impl(const std::string &directory) : weights(directory + "/model.safetensors") {
        // safetensors header and tensor spans (src/exl3_model.cpp:79-112)
        uint64_t header_size = 0;
        for (unsigned i = 0; i < 8; ++i) header_size |= uint64_t(weights.data[i]) << (i * 8);
        if (header_size > 64 * 1024 * 1024 || header_size > weights.size - 8)
            throw std::runtime_error("Invalid safetensors header length");
        const char *hb = reinterpret_cast<const char *>(weights.data + 8);
        const Value header = exl3json::parse(hb, hb + header_size);
        if (!header.is_object()) throw std::runtime_error("Invalid safetensors header");
        const size_t data_begin = 8 + (size_t)header_size;
        std::vector<std::pair<size_t, size_t>> spans;
        static const std::map<std::string, size_t> widths = {{"F16", 2}, {"BF16", 2}, {"I16", 2}, {"F32", 4}, {"I32", 4}};
        for (const auto &member : header.members) {
            if (member.first == "__metadata__") continue;
            const Value &info = member.second;
            Tensor t;
            t.dtype = string_of(info.at("dtype"));
            auto width = widths.find(t.dtype);
            if (width == widths.end()) throw std::runtime_error("Unsupported model dtype");
            size_t elements = 1;
            for (const Value *dimension : elements_of(info.at("shape"))) {
                const size_t dim = positive_integer(*dimension);
                if (elements > std::numeric_limits<size_t>::max() / dim) throw std::runtime_error("Tensor shape overflow");
                elements *= dim;
                t.shape.push_back(dim);
            }
            const Value &offsets = info.at("data_offsets");
            if (!offsets.is_array() || offsets.items.size() != 2) throw std::runtime_error("Invalid tensor offset pair");
            const size_t begin = positive_integer(offsets.items[0], true), end = positive_integer(offsets.items[1], true);
            if (end < begin || end > weights.size - data_begin ||
                elements > std::numeric_limits<size_t>::max() / width->second || end - begin != elements * width->second)
                throw std::runtime_error("Invalid tensor data span");
            t.data = weights.data + data_begin + begin;
            t.size = end - begin;
            tensors.emplace(member.first, std::move(t));
            spans.emplace_back(begin, end);
        }
        std::sort(spans.begin(), spans.end());
        for (auto span : spans) {
            if (span.first != payload) throw std::runtime_error("Overlapping or missing tensor data");
            payload = span.second;
        }
        if (payload != weights.size - data_begin) throw std::runtime_error("Unaccounted model payload");

        // deployment manifest (src/exl3_model.cpp:113-131)
        std::ifstream manifest_file(directory + "/hexagon-exl3.json", std::ios::binary);
        const std::string text((std::istreambuf_iterator<char>(manifest_file)), std::istreambuf_iterator<char>());
        const Value manifest = exl3json::parse(text.data(), text.data() + text.size());
        if (!manifest.at("format").equals("hexagon-exl3") || !manifest.at("version").equals(1) ||
            !manifest.at("kv_cache").equals("f16"))
            throw std::runtime_error("Unsupported deployment manifest");
        const Value &embedding = manifest.at("input_embedding");
        if (!embedding.at("type").equals("tied_linear") || !embedding.at("basis").equals("original") ||
            !embedding.at("token_axis").equals(1))
            throw std::runtime_error("Unsupported embedding alias");
        k = positive_integer(embedding.at("hidden_size"));
        n = positive_integer(embedding.at("vocab_size"));
        if (k % 128 || n % 128 || k > 16384 || n > 1048576) throw std::runtime_error("Invalid embedding geometry");
        parameters = positive_integer(manifest.at("reference_parameter_count"));
        if (positive_integer(manifest.at("weight_payload_bytes")) != payload || double(payload) * 8 / parameters > 5.0)
            throw std::runtime_error("Model payload or budget mismatch");

        // the tied head (src/exl3_model.cpp:132-156)
        head_prefix = string_of(embedding.at("source"));
        const Tensor &packed = tensor(head_prefix + ".trellis");
        if (packed.dtype != "I16" || packed.shape.size() != 3 || packed.shape[0] != k / 16 || packed.shape[1] != n / 16 ||
            packed.shape[2] % 16 || packed.shape[2] < 16 || packed.shape[2] > 128)
            throw std::runtime_error("Invalid head trellis");
        head_bits = unsigned(packed.shape[2] / 16);
        for (const auto &entry : {std::make_pair("suh", k), std::make_pair("svh", n)}) {
            const Tensor &scale = tensor(head_prefix + "." + entry.first);
            if (scale.dtype != "F16" || scale.shape != std::vector<size_t>{entry.second})
                throw std::runtime_error("Invalid head scale");
        }
        head_codebook = codebook_of(head_prefix);
    }

    // the 128 columns [128 group, +128) of the head's original-basis weights,
    // [k][128] fp16 bits, by exl3_hip_reconstruct on the head's device
    void reconstruct_group(size_t group, uint16_t *out) const {
        if (head_device < 0) {
            int dev = 0;
            hip_check(hipGetDevice(&dev), "hipGetDevice");
            const Tensor &p = tensor(head_prefix + ".trellis"), &su = tensor(head_prefix + ".suh"),
                         &sv = tensor(head_prefix + ".svh");
            auto t = std::make_unique<DeviceBuffer>(p.size), s = std::make_unique<DeviceBuffer>(su.size),
                 v = std::make_unique<DeviceBuffer>(sv.size), b = std::make_unique<DeviceBuffer>(k * 128 * 2);
            hip_check(hipMemcpy(t->ptr, p.data, p.size, hipMemcpyHostToDevice), "hipMemcpy H2D");
            hip_check(hipMemcpy(s->ptr, su.data, su.size, hipMemcpyHostToDevice), "hipMemcpy H2D");
            hip_check(hipMemcpy(v->ptr, sv.data, sv.size, hipMemcpyHostToDevice), "hipMemcpy H2D");
            d_trellis = std::move(t);
            d_su = std::move(s);
            d_sv = std::move(v);
            d_block = std::move(b);
            head_device = dev;
        }
        DeviceScope scope(head_device);
        const exl3_status st = exl3_hip_reconstruct(
            d_trellis->ptr, EXL3_LAYOUT_UPSTREAM_TILES, static_cast<const uint16_t *>(d_su->ptr),
            static_cast<const uint16_t *>(d_sv->ptr), head_bits, (unsigned)head_codebook, k, n, group * 128, 128,
            static_cast<uint16_t *>(d_block->ptr), nullptr);
        if (st != EXL3_OK) throw std::runtime_error(std::string("exl3_hip_reconstruct: ") + exl3_hip_status_string(st));
        hip_check(hipMemcpy(out, d_block->ptr, k * 128 * 2, hipMemcpyDeviceToHost), "hipMemcpy D2H");
    }
};

Model::Model(const std::string &directory) : impl(std::make_unique<Impl>(directory)) {}
Model::~Model() = default;
size_t Model::tensor_count() const { return impl->tensors.size(); }
size_t Model::payload_bytes() const { return impl->payload; }
size_t Model::hidden_size() const { return impl->k; }
size_t Model::vocab_size() const { return impl->n; }
double Model::bits_per_weight() const { return double(impl->payload) * 8 / impl->parameters; }

// src/exl3_model.cpp:168-187: column token % 128 of the reconstructed 128-token
// group, groups kept in a 16-entry most-recently-used list
std::vector<uint16_t> Model::embedding(uint32_t token) const {
    if (token >= impl->n) throw std::invalid_argument("Token ID outside vocabulary");
    const size_t group = token / 128;
    std::lock_guard<std::mutex> guard(impl->cache_mutex);
    auto &cache = impl->cache;
    auto entry = std::find_if(cache.begin(), cache.end(), [&](const auto &item) { return item.first == group; });
    if (entry == cache.end()) {
        auto block = std::make_shared<std::vector<uint16_t>>(impl->k * 128);
        impl->reconstruct_group(group, block->data());
        cache.emplace_front(group, std::move(block));
        if (cache.size() > 16) cache.pop_back();
    } else {
        cache.splice(cache.begin(), cache, entry);
    }
    const auto &block = *cache.front().second;
    std::vector<uint16_t> result(impl->k);
    for (size_t row = 0; row < impl->k; ++row) result[row] = block[row * 128 + token % 128];
    return result;
}

std::vector<Model::Matrix> Model::matrices() const {
    std::vector<Matrix> out;
    const std::string suffix = ".trellis";
    for (const auto &entry : impl->tensors) {
        const std::string &name = entry.first;
        if (name.size() <= suffix.size() || name.compare(name.size() - suffix.size(), suffix.size(), suffix)) continue;
        const Tensor &t = entry.second;
        if (t.dtype != "I16" || t.shape.size() != 3 || t.shape[2] % 16 || t.shape[2] < 16 || t.shape[2] > 128) continue;
        const std::string prefix = name.substr(0, name.size() - suffix.size());
        const size_t k = t.shape[0] * 16, n = t.shape[1] * 16;
        auto su = impl->tensors.find(prefix + ".suh"), sv = impl->tensors.find(prefix + ".svh");
        if (su == impl->tensors.end() || sv == impl->tensors.end()) continue;
        if (su->second.dtype != "F16" || su->second.shape != std::vector<size_t>{k} || sv->second.dtype != "F16" ||
            sv->second.shape != std::vector<size_t>{n})
            continue;
        out.push_back({prefix, unsigned(t.shape[2] / 16), impl->codebook_of(prefix), k, n});
    }
    return out;
}

size_t Model::record_bytes(const Matrix &m) const { return (m.n / 128) * (m.k / 128) * (2048 * (size_t)m.bits + 512); }

void Model::upload_records(const Matrix &m, void *records, hipStream_t stream) const {
    if (m.k % 128 || m.n % 128 || m.bits < 1 || m.bits > 8)
        throw std::invalid_argument("Group records need k and n multiples of 128");
    const Tensor &p = impl->tensor(m.prefix + ".trellis"), &su = impl->tensor(m.prefix + ".suh"),
                 &sv = impl->tensor(m.prefix + ".svh");
    if (p.size != m.k * m.n * m.bits / 8 || su.size != 2 * m.k || sv.size != 2 * m.n)
        throw std::invalid_argument("Matrix does not match the model's tensors");
    DeviceBuffer dp(p.size), ds(su.size), dv(sv.size);
    hip_check(hipMemcpyAsync(dp.ptr, p.data, p.size, hipMemcpyHostToDevice, stream), "hipMemcpyAsync H2D");
    hip_check(hipMemcpyAsync(ds.ptr, su.data, su.size, hipMemcpyHostToDevice, stream), "hipMemcpyAsync H2D");
    hip_check(hipMemcpyAsync(dv.ptr, sv.data, sv.size, hipMemcpyHostToDevice, stream), "hipMemcpyAsync H2D");
    const exl3_status st = exl3_hip_pack_records(static_cast<const uint16_t *>(dp.ptr), static_cast<const uint16_t *>(ds.ptr),
                                                 static_cast<const uint16_t *>(dv.ptr), m.bits, m.k, m.n, records, stream);
    if (st == EXL3_INVAL_PARAMS) throw std::invalid_argument("exl3_hip_pack_records: invalid parameters");
    if (st != EXL3_OK) throw std::runtime_error(std::string("exl3_hip_pack_records: ") + exl3_hip_status_string(st));
    hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize");  // before the staging buffers are freed
}

}  // namespace exl3

// ------------------------------------------------------------------ C wrappers
struct exl3_model {
    exl3::Model model;
    std::vector<exl3::Model::Matrix> matrices;
    explicit exl3_model(const char *directory) : model(directory), matrices(model.matrices()) {}
};

namespace {
void set_error(char *error, size_t bytes, const char *what) {
    if (!error || !bytes) return;
    std::strncpy(error, what, bytes - 1);
    error[bytes - 1] = '\0';
}
}  // namespace

extern "C" {

exl3_model *exl3_hip_model_open(const char *directory, char *error, size_t error_bytes) {
    if (!directory) {
        set_error(error, error_bytes, "NULL directory");
        return nullptr;
    }
    try {
        return new exl3_model(directory);
    } catch (const std::exception &e) {
        set_error(error, error_bytes, e.what());
    } catch (...) {
        set_error(error, error_bytes, "unknown error");
    }
    return nullptr;
}

void exl3_hip_model_close(exl3_model *m) { delete m; }

size_t exl3_hip_model_tensor_count(const exl3_model *m) { return m ? m->model.tensor_count() : 0; }
size_t exl3_hip_model_payload_bytes(const exl3_model *m) { return m ? m->model.payload_bytes() : 0; }
size_t exl3_hip_model_hidden_size(const exl3_model *m) { return m ? m->model.hidden_size() : 0; }
size_t exl3_hip_model_vocab_size(const exl3_model *m) { return m ? m->model.vocab_size() : 0; }
double exl3_hip_model_bits_per_weight(const exl3_model *m) { return m ? m->model.bits_per_weight() : 0.0; }

exl3_status exl3_hip_model_embedding(const exl3_model *m, uint32_t token, uint16_t *out) {
    if (!m || !out) return EXL3_INVAL_PARAMS;
    try {
        const std::vector<uint16_t> row = m->model.embedding(token);
        std::memcpy(out, row.data(), row.size() * 2);
        return EXL3_OK;
    } catch (const std::invalid_argument &) {
        return EXL3_INVAL_PARAMS;
    } catch (...) {
        return EXL3_HIP_ERROR;
    }
}

size_t exl3_hip_model_matrix_count(const exl3_model *m) { return m ? m->matrices.size() : 0; }

exl3_status exl3_hip_model_matrix(const exl3_model *m, size_t index, char *name, size_t name_bytes, unsigned *bits,
                                  unsigned *codebook, size_t *k, size_t *n) {
    if (!m || index >= m->matrices.size()) return EXL3_INVAL_PARAMS;
    const auto &x = m->matrices[index];
    set_error(name, name_bytes, x.prefix.c_str());
    if (bits) *bits = x.bits;
    if (codebook) *codebook = (unsigned)x.codebook;
    if (k) *k = x.k;
    if (n) *n = x.n;
    return EXL3_OK;
}

size_t exl3_hip_model_record_bytes(const exl3_model *m, size_t index) {
    if (!m || index >= m->matrices.size()) return 0;
    return m->model.record_bytes(m->matrices[index]);
}

exl3_status exl3_hip_model_upload_records(const exl3_model *m, size_t index, void *records, hipStream_t stream) {
    if (!m || index >= m->matrices.size() || !records || (uintptr_t)records % 16) return EXL3_INVAL_PARAMS;
    try {
        m->model.upload_records(m->matrices[index], records, stream);
        return EXL3_OK;
    } catch (const std::invalid_argument &) {
        return EXL3_INVAL_PARAMS;
    } catch (...) {
        return EXL3_HIP_ERROR;
    }
}

}  // extern "C"
