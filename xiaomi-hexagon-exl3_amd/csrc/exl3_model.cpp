// exl3_model.cpp -- exl3::Model (include/exl3_model.h) over the host-side
// format passes of exl3_model_format.hpp: the tied-embedding reconstruct and
// the record packing run on the GPU through the C-ABI.  Also the C wrappers
// exl3_hip_model_* of include/exl3_hip.h.
#include "exl3_model.h"

#include <hip/hip_runtime.h>

#include <array>
#include <cstring>
#include <limits>
#include <mutex>
#include <stdexcept>
#include <utility>

#include "exl3_hip.h"
#include "exl3_model_format.hpp"

namespace exl3 {
namespace {

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
    template <typename T>
    T *as() const { return static_cast<T *>(ptr); }
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

// Host copies of reconstructed 128-token column groups of the head: the
// kSlots most recently used ones (the reference keeps 16,
// src/exl3_model.cpp:168-187).  Each slot carries the tick of its last use; a
// miss refills the slot used longest ago (an empty slot first).
class GroupCache {
public:
    static constexpr size_t kSlots = 16;

    template <typename Fill>
    const std::vector<uint16_t> &block(size_t group, size_t elements, Fill &&fill) {
        Slot *victim = &slots_[0];
        for (Slot &s : slots_) {
            if (s.group == group) {
                s.tick = ++clock_;
                return s.data;
            }
            if (s.tick < victim->tick) victim = &s;
        }
        victim->group = kEmpty;  // stays empty if fill throws
        victim->data.resize(elements);
        fill(victim->data.data());
        victim->group = group;
        victim->tick = ++clock_;
        return victim->data;
    }

private:
    static constexpr size_t kEmpty = std::numeric_limits<size_t>::max();
    struct Slot {
        size_t group = kEmpty;
        uint64_t tick = 0;
        std::vector<uint16_t> data;
    };
    std::array<Slot, kSlots> slots_;
    uint64_t clock_ = 0;
};

// The head's trellis and scales on the device that made the first embedding
// call, and a [k][128] output block for exl3_hip_reconstruct.
struct DeviceHead {
    int device = -1;
    DeviceBuffer trellis, su, sv, block;

    void upload(const exl3fmt::OpenedModel &om) {
        const std::string &h = om.manifest.head;
        const exl3fmt::TensorEntry *parts[3] = {&om.index.get(h + ".trellis"), &om.index.get(h + ".suh"),
                                                &om.index.get(h + ".svh")};
        DeviceBuffer *dst[3] = {&trellis, &su, &sv};
        int dev = 0;
        hip_check(hipGetDevice(&dev), "hipGetDevice");
        for (int i = 0; i < 3; ++i) {
            DeviceBuffer fresh(parts[i]->bytes);
            hip_check(hipMemcpy(fresh.ptr, om.file.bytes() + om.index.payload_begin + parts[i]->offset,
                                parts[i]->bytes, hipMemcpyHostToDevice),
                      "hipMemcpy H2D");
            std::swap(dst[i]->ptr, fresh.ptr);
        }
        DeviceBuffer out(om.manifest.hidden * 128 * 2);
        std::swap(block.ptr, out.ptr);
        device = dev;
    }
};

}  // namespace

struct Model::Impl {
    exl3fmt::OpenedModel om;
    mutable std::mutex mu;  // guards the cache and the device head
    mutable GroupCache cache;
    mutable DeviceHead head;

    explicit Impl(const std::string &directory) : om(exl3fmt::open_model(directory)) {}

    const uint8_t *payload(const exl3fmt::TensorEntry &e) const {
        return om.file.bytes() + om.index.payload_begin + e.offset;
    }

    // columns [128 group, +128) of the head's original-basis weights as
    // [k][128] fp16 bits, reconstructed on the head's device
    void reconstruct_group(size_t group, uint16_t *out) const {
        if (head.device < 0) head.upload(om);
        DeviceScope scope(head.device);
        const size_t k = om.manifest.hidden, n = om.manifest.vocab;
        const exl3_status st =
            exl3_hip_reconstruct(head.trellis.ptr, EXL3_LAYOUT_UPSTREAM_TILES, head.su.as<const uint16_t>(),
                                 head.sv.as<const uint16_t>(), om.head.bits, (unsigned)om.head.codebook, k, n,
                                 group * 128, 128, head.block.as<uint16_t>(), nullptr);
        if (st != EXL3_OK) throw std::runtime_error(std::string("exl3_hip_reconstruct: ") + exl3_hip_status_string(st));
        hip_check(hipMemcpy(out, head.block.ptr, k * 128 * 2, hipMemcpyDeviceToHost), "hipMemcpy D2H");
    }
};

Model::Model(const std::string &directory) : impl(std::make_unique<Impl>(directory)) {}
Model::~Model() = default;

size_t Model::tensor_count() const { return impl->om.index.entries.size(); }
size_t Model::payload_bytes() const { return impl->om.index.payload_bytes; }
size_t Model::hidden_size() const { return impl->om.manifest.hidden; }
size_t Model::vocab_size() const { return impl->om.manifest.vocab; }
double Model::bits_per_weight() const {
    return double(impl->om.index.payload_bytes) * 8 / double(impl->om.manifest.parameters);
}

// Token t's row is column t % 128 of its group's reconstruct (the tied head read
// along its output axis, src/exl3_model.cpp:168-187).
std::vector<uint16_t> Model::embedding(uint32_t token) const {
    const size_t k = impl->om.manifest.hidden;
    if (token >= impl->om.manifest.vocab) throw std::invalid_argument("Token ID outside vocabulary");
    std::lock_guard<std::mutex> lock(impl->mu);
    const std::vector<uint16_t> &group = impl->cache.block(
        token / 128, k * 128, [&](uint16_t *out) { impl->reconstruct_group(token / 128, out); });
    std::vector<uint16_t> row(k);
    const size_t column = token % 128;
    for (size_t r = 0; r < k; ++r) row[r] = group[r * 128 + column];
    return row;
}

std::vector<Model::Matrix> Model::matrices() const {
    std::vector<Matrix> out;
    for (const exl3fmt::MatrixEntry &e : exl3fmt::list_matrices(impl->om.index, impl->om.file.bytes()))
        out.push_back({e.prefix, e.bits, static_cast<Codebook>(e.codebook), e.k, e.n});
    return out;
}

std::vector<Model::EmbeddingTable> Model::embedding_tables() const {
    std::vector<EmbeddingTable> out;
    for (const exl3fmt::EmbeddingTableEntry &e : exl3fmt::list_embedding_tables(impl->om.index))
        out.push_back({e.prefix, e.rows, e.groups, e.width_padded, e.bits});
    return out;
}

size_t Model::record_bytes(const Matrix &m) const { return (m.n / 128) * (m.k / 128) * (2048 * (size_t)m.bits + 512); }

void Model::upload_records(const Matrix &m, void *records, hipStream_t stream) const {
    if (m.k % 128 || m.n % 128 || m.bits < 1 || m.bits > 8)
        throw std::invalid_argument("Group records need k and n multiples of 128");
    const exl3fmt::TensorIndex &ix = impl->om.index;
    const exl3fmt::TensorEntry *src[3] = {&ix.get(m.prefix + ".trellis"), &ix.get(m.prefix + ".suh"),
                                          &ix.get(m.prefix + ".svh")};
    const size_t want[3] = {m.k * m.n * m.bits / 8, 2 * m.k, 2 * m.n};
    for (int i = 0; i < 3; ++i)
        if (src[i]->bytes != want[i]) throw std::invalid_argument("Matrix does not match the model's tensors");
    // staging copies of the upstream tensors, packed into records on the device
    DeviceBuffer staged[3] = {DeviceBuffer(want[0]), DeviceBuffer(want[1]), DeviceBuffer(want[2])};
    for (int i = 0; i < 3; ++i)
        hip_check(hipMemcpyAsync(staged[i].ptr, impl->payload(*src[i]), want[i], hipMemcpyHostToDevice, stream),
                  "hipMemcpyAsync H2D");
    const exl3_status st = exl3_hip_pack_records(staged[0].as<const uint16_t>(), staged[1].as<const uint16_t>(),
                                                 staged[2].as<const uint16_t>(), m.bits, m.k, m.n, records, stream);
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

exl3_status exl3_hip_model_embedding_tables(const exl3_model *m, size_t *count, char *error, size_t error_bytes) {
    if (!m || !count) return EXL3_INVAL_PARAMS;
    try {
        *count = m->model.embedding_tables().size();
        return EXL3_OK;
    } catch (const std::exception &e) {
        set_error(error, error_bytes, e.what());
        return EXL3_INVAL_PARAMS;
    }
}

exl3_status exl3_hip_model_embedding_table(const exl3_model *m, size_t index, char *name, size_t name_bytes,
                                           size_t *rows, size_t *groups, unsigned *bits, size_t *width_padded) {
    if (!m) return EXL3_INVAL_PARAMS;
    try {
        const std::vector<exl3::Model::EmbeddingTable> tables = m->model.embedding_tables();
        if (index >= tables.size()) return EXL3_INVAL_PARAMS;
        const exl3::Model::EmbeddingTable &t = tables[index];
        set_error(name, name_bytes, t.prefix.c_str());
        if (rows) *rows = t.rows;
        if (groups) *groups = t.groups;
        if (bits) *bits = t.bits;
        if (width_padded) *width_padded = t.width_padded;
        return EXL3_OK;
    } catch (const std::exception &) {
        return EXL3_INVAL_PARAMS;
    }
}

}  // extern "C"
