// exl3_launch.hpp -- internal launcher interface between the C-ABI (exl3_api.cpp)
// and the gfx950 kernels (exl3_kernels.hip).  Launchers assume the caller has
// validated every argument; they only enqueue work and return hipGetLastError().
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace exl3k {

// GEMV: hi/lo fp16 halves of 8 rows per 16 MFMA columns (one block up to 8 rows, two
// up to 16); 17..32 rows as two blocks of 16 fp16 rows prepared once per call.
// A single matrix above kGemvSingleMaxRows rows runs the GEMM (32-row tiles up to
// 32 rows), which is flat in the row count from there (k = 14336, n = 4096:
// 21.2-21.5 us for rows 14..32, against the GEMV's 21.4 at 14 rows, 22.4 at 16,
// 24.5 at 20), except at 15..16 rows when a GEMV workgroup's prep is at most
// kGemvSinglePrepBlocks (record, row) blocks: there the hi/lo GEMV is faster
// (rows 16: k = 2048, n = 2048, 6 bits 10.4 against 13.6 us; k = 2048, n = 6144
// 12.0 against 13.8; k = 6144, n = 2048, 3 bits 12.4 against 14.5), at k = 14336
// it is not (22.3 against 21.5-21.8 us, 112 blocks).  A grouped call keeps its
// one GEMV launch up to kGemvMaxRows rows (q/k/v at 32 rows: 18 us against 41 us
// for three GEMM calls).
constexpr int kGemvMaxRows = 32;
constexpr int kGemvSingleMaxRows = 14;
constexpr int kGemvSinglePrepBlocks = 64;
constexpr int kGemvWaves = 8;     // waves per GEMV workgroup (a multiple of 4)

// Every plan starts with the same region, which only the GEMV's split-K hand-off
// touches: the exchange, kGemvExchangeBytes of 32-bit words carrying split
// partials.  It is zero before a workspace's first use, every GEMV call leaves
// it zero again (the workgroup that sums a column group's partials clears what
// it consumed) and no other kernel writes it.  One workspace therefore serves
// calls of any shape and row count in turn, when it is as large as each needs.
// A GEMV whose partials would not fit the exchange runs as a GEMM instead.  The
// GEMM splits k only while it has fewer than kGemmSplitTiles output tiles; a
// second kernel sums its split partials.
constexpr size_t kGemmSplitTiles = 512;
constexpr size_t kGemvExchangeBytes = (size_t)16 << 20;
// Right after the exchange: the status word (32 bits, in a 256-byte block).
// Zero while the exchange can be trusted.  A workgroup that gives up waiting for
// a split's partial (a bounded wait that ran out) sets it to 1; from then on a
// partial stored late may sit in the exchange, so every later GEMV call with
// that workspace writes NaN for every output it sums, without waiting, until
// the workspace is zero-filled again (exl3_hip_workspace_init).
constexpr size_t kStatusOffset = kGemvExchangeBytes;
constexpr size_t kStatusBytes = 256;
// bytes every workspace starts with: the exchange and the status block
constexpr size_t kSharedPrefixBytes = kGemvExchangeBytes + kStatusBytes;

// Failure injection for tests of the give-up path (never set by a product
// caller): spin_limit > 0 replaces the wait budget of the split-K hand-off (in
// polls per wave); drop_split >= 0 makes that split's workgroups skip storing
// their partial.  set_exchange_fault(0, -1) restores the defaults.
void set_exchange_fault(int spin_limit, int drop_split);
int exchange_spin_limit();   // the wait budget of the split-K hand-off (polls per wave)
int exchange_drop_split();   // -1 unless a test dropped a split

// Up to kGemvMaxTargets matrices that share k, the bit rate, the codebook and x,
// served by one GEMV launch: column groups [nb_end[i-1], nb_end[i]) belong to
// matrix i (records[i], output y[i] with row stride y_stride[i] elements).
constexpr int kGemvMaxTargets = 4;
struct GemvTargets {
    const uint8_t *records[kGemvMaxTargets];
    void *y[kGemvMaxTargets];
    size_t y_stride[kGemvMaxTargets];
    const void *res[kGemvMaxTargets];  // optional residual added to y (y's dtype), or null
    size_t res_stride[kGemvMaxTargets];
    int nb_end[kGemvMaxTargets];
    int count;
};

// Whole matrices of one rate decoded by one launch (decode_batch_kernel).
constexpr int kDecodeBatchMax = 32;
// 256-column decode blocks per workgroup of a batch launch (even)
constexpr unsigned kDecodeBlocksPerWg = 2;
struct DecodeBatch {
    const void *src[kDecodeBatchMax];
    uint16_t *out[kDecodeBatchMax];
    size_t k[kDecodeBatchMax], n[kDecodeBatchMax];
    unsigned wg_begin[kDecodeBatchMax];  // first workgroup of each matrix: ceil((k/16) ceil(n/256) / kDecodeBlocksPerWg) each
    int count;
};

struct GemvPlan {
    int nbs, kbs, splits, nkw;  // nkw: largest kb count of a split
    size_t partials_off, exchange_bytes, dummy_off, xpre_off, bytes;
    bool fits;  // the partials fit the exchange (else the call runs as a GEMM)
};
struct GemmPlan {
    int nbs, kbs, bm, mtiles, splits;  // bm: rows per workgroup tile (128, 256 or 512)
    size_t xh_off, partials_off, exps_off, bytes;
};

GemvPlan gemv_plan(size_t k, size_t n, size_t rows);
// rows <= kGemvMaxRows and the GEMV's split partials fit the exchange
bool gemv_serves(size_t k, size_t n, size_t rows);
// the GEMV for one matrix: up to kGemvSingleMaxRows rows, and at 15..16 rows where
// a workgroup preps at most kGemvSinglePrepBlocks (record, row) blocks
bool gemv_serves_single(size_t k, size_t n, size_t rows);
GemmPlan gemm_plan(size_t k, size_t n, size_t rows);
int gemm_tile_rows(size_t rows);

// res (optional, y's dtype, row stride res_stride): y = res + layer(x), the sum
// rounded once; res may be y itself (same stride)
hipError_t launch_gemv(const void *records, int bits, int cb, size_t k, size_t n, const void *x, int x_f16,
                       size_t rows, size_t x_stride, void *y, int y_f16, size_t y_stride, void *workspace,
                       const GemvPlan &plan, hipStream_t stream, const void *res = nullptr, size_t res_stride = 0);
hipError_t launch_gemv_targets(const GemvTargets &targets, int bits, int cb, const void *x, int x_f16, size_t rows,
                               size_t x_stride, int y_f16, void *workspace, const GemvPlan &plan, hipStream_t stream);
hipError_t launch_gemm(const void *records, int bits, int cb, size_t k, size_t n, const void *x, int x_f16,
                       size_t rows, size_t x_stride, void *y, int y_f16, size_t y_stride, void *workspace,
                       const GemmPlan &plan, hipStream_t stream, const void *res = nullptr, size_t res_stride = 0);
hipError_t launch_decode(const void *src, int records_layout, int bits, int cb, size_t k, size_t n,
                         size_t first, size_t count, uint16_t *out, hipStream_t stream);
hipError_t launch_decode_batch(const DecodeBatch &batch, int records_layout, int bits, int cb, unsigned workgroups,
                               hipStream_t stream);
hipError_t launch_reconstruct(const void *src, int records_layout, const uint16_t *su, const uint16_t *sv,
                              int bits, int cb, size_t k, size_t n, size_t first, size_t count, uint16_t *out,
                              hipStream_t stream);
// ids[i * ids_stride] for i < count (ids_stride in int32 elements, may be 0)
hipError_t launch_get_rows(const void *records, int bits, int cb, size_t k, size_t n, const int32_t *ids,
                           size_t ids_stride, size_t count, void *out, int out_f16, size_t out_stride, int *bad_ids,
                           hipStream_t stream);
hipError_t launch_codebook(const uint16_t *states, size_t count, int cb, uint16_t *out, hipStream_t stream);
hipError_t launch_hadamard(float *values, size_t count, hipStream_t stream);
hipError_t launch_pack_records(const uint16_t *packed, const uint16_t *su, const uint16_t *sv, int bits, size_t k,
                               size_t n, void *records, hipStream_t stream);
hipError_t launch_validate(const void *records, size_t nrecords, int bits, int *result, hipStream_t stream);
hipError_t launch_zero(void *ptr, size_t bytes, hipStream_t stream);

}  // namespace exl3k
