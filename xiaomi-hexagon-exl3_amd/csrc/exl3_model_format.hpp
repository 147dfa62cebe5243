// exl3_model_format.hpp -- host-only reading and validation of an EXL3
// deployment model directory (model.safetensors + hexagon-exl3.json), in four
// passes that each produce a plain value:
//
//   1. WeightFile            the weights, mapped read-only
//   2. TensorIndex           the safetensors header parsed into tensor entries,
//                            then checked as a whole: the spans tile the payload
//   3. Manifest              the deployment manifest's fields, format-checked
//   4. HeadBinding           the manifest's tied head resolved in the index:
//                            payload budget, trellis / scale shapes, codebook
//
// The checks and exception messages are those of the reference reader
// (src/exl3_model.cpp:22-156): callers and tests match on them.  Nothing here
// touches the GPU, so the format code builds alone (with sanitizers, for tests).
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

namespace exl3fmt {

// ---- pass 1: the weight file
class WeightFile {
public:
    // throws std::runtime_error: "Cannot open model weights", "Invalid weight
    // file size" (shorter than the 8-byte length prefix), "Cannot map model weights"
    static WeightFile map(const std::string &path);
    const uint8_t *bytes() const { return base_.get(); }
    size_t size() const { return size_; }

private:
    std::shared_ptr<const uint8_t> base_;  // unmapped by its deleter
    size_t size_ = 0;
};

// ---- pass 2: tensor index
enum class DType : uint8_t { F16, BF16, I16, F32, I32 };
size_t dtype_bytes(DType t);
const char *dtype_name(DType t);

struct TensorEntry {
    std::string name;
    DType dtype = DType::F16;
    std::vector<size_t> dims;   // empty for a scalar
    size_t offset = 0;          // from the start of the payload
    size_t bytes = 0;
    bool is(DType t, std::initializer_list<size_t> shape) const;
};

struct TensorIndex {
    size_t payload_begin = 0;   // file offset of the payload (8 + header length)
    size_t payload_bytes = 0;
    std::vector<TensorEntry> entries;   // sorted by name
    const TensorEntry *find(const std::string &name) const;
    // throws "Missing model tensor: <name>"
    const TensorEntry &get(const std::string &name) const;
};

// Parses the header and checks every entry (dtype, positive integer dims,
// offset pair matching the shape, inside the payload), then the spans as a set
// (they cover the payload exactly, without overlap).
TensorIndex index_tensors(const uint8_t *file, size_t file_bytes);

// ---- pass 3: manifest
struct Manifest {
    std::string head;           // tensor prefix of the tied input embedding
    size_t hidden = 0, vocab = 0;
    size_t parameters = 0;      // reference_parameter_count
    size_t payload_bytes = 0;   // weight_payload_bytes
};
Manifest read_manifest(const std::string &json_text);

// ---- pass 4: the tied head
struct HeadBinding {
    unsigned bits = 0;
    int codebook = 0;           // exl3::Codebook value
};
// Manifest against index: payload size and the 5.0 bits-per-weight budget,
// then the head's trellis and scales and its codebook marker.
HeadBinding bind_head(const TensorIndex &index, const uint8_t *file, const Manifest &manifest);

// Codebook named by <prefix>.mul1 / <prefix>.mcg (I32 scalar multipliers),
// three_inst (0) when neither exists.  Throws on an ambiguous or wrong marker.
int codebook_of(const TensorIndex &index, const uint8_t *file, const std::string &prefix);

// Every <prefix>.trellis (I16, [k/16, n/16, 16*bits], bits 1..8) whose .suh
// ([k] F16) and .svh ([n] F16) exist, in name order.
struct MatrixEntry {
    std::string prefix;
    unsigned bits = 0;
    int codebook = 0;
    size_t k = 0, n = 0;
};
std::vector<MatrixEntry> list_matrices(const TensorIndex &index, const uint8_t *file);

// Row-coded EXL3 embedding tables: every <prefix>.trellis of rank 2 with a
// <prefix>.signs, checked as the reference's model audit checks them
// (tools/inspect_model.py:78-90); throws std::runtime_error with its messages.
struct EmbeddingTableEntry {
    std::string prefix;
    size_t rows = 0, groups = 0, width_padded = 0;
    unsigned bits = 0;
};
std::vector<EmbeddingTableEntry> list_embedding_tables(const TensorIndex &index);

// The whole directory through passes 1-4 (what exl3::Model's constructor does
// before any device work).
struct OpenedModel {
    WeightFile file;
    TensorIndex index;
    Manifest manifest;
    HeadBinding head;
};
OpenedModel open_model(const std::string &directory);

}  // namespace exl3fmt
