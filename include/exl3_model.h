/*
 * exl3_model.h -- the EXL3 deployment-model reader: the same class, names,
 * argument meaning and exceptions as the reference's include/exl3_model.h
 * (exl3::Model, src/exl3_model.cpp:79-187), plus the device accessors this
 * library adds for the GPU layer (marked below).
 *
 * A model directory holds model.safetensors (EXL3 tensors: <prefix>.trellis I16
 * [k/16, n/16, 16*bits], <prefix>.suh F16 [k], <prefix>.svh F16 [n], optional
 * <prefix>.mul1 / <prefix>.mcg I32 codebook markers) and hexagon-exl3.json (the
 * deployment manifest).  The constructor maps the weights read-only and
 * validates them as the reference does; malformed input throws
 * std::runtime_error.  embedding() runs the reconstruct on the current HIP
 * device (bit-exact with exl3::reconstruct_slice) and keeps the 16 most recent
 * 128-token groups on the host, as the reference does.
 */
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include <hip/hip_runtime_api.h>

#include "exl3_codec.h"

namespace exl3 {

class Model {
public:
    explicit Model(const std::string & directory);
    ~Model();
    Model(const Model &) = delete;
    Model & operator=(const Model &) = delete;
    size_t tensor_count() const;
    size_t payload_bytes() const;
    size_t hidden_size() const;
    size_t vocab_size() const;
    double bits_per_weight() const;
    std::vector<uint16_t> embedding(uint32_t token) const;

    /* ---- added by this library: EXL3 matrices for the GPU layer ---- */
    struct Matrix {
        std::string prefix;   /* tensor-name prefix, e.g. "model.layers.0.mlp.down_proj" */
        unsigned bits;        /* 1..8, from the trellis shape */
        Codebook codebook;    /* from the .mul1 / .mcg marker, else three_inst */
        size_t k, n;          /* input and output features */
    };
    /* every <prefix>.trellis of rank 3 with its .suh and .svh, in name order */
    std::vector<Matrix> matrices() const;
    /* device bytes of the group records of one matrix: (n/128)*(k/128)*(2048*bits+512) */
    size_t record_bytes(const Matrix & matrix) const;
    /* pack one matrix into group records (include/exl3-block.h) at device
     * pointer `records` (16-byte aligned, record_bytes() long) on `stream`;
     * returns after the records are complete.  k and n must be multiples of 128. */
    void upload_records(const Matrix & matrix, void * records, hipStream_t stream) const;
    /* row-coded embedding tables (<prefix>.trellis [rows, groups * (16 bits + 1)] I16
     * with <prefix>.signs [groups, 256] F16), validated as the reference's model
     * audit does (tools/inspect_model.py:78-90); malformed tables throw
     * std::runtime_error.  Listing only: their decode is not implemented. */
    struct EmbeddingTable {
        std::string prefix;
        size_t rows, groups, width_padded;
        unsigned bits;
    };
    std::vector<EmbeddingTable> embedding_tables() const;

private:
    struct Impl;
    std::unique_ptr<Impl> impl;
};

} // namespace exl3
