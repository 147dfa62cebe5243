// exl3_api.cpp -- the C-ABI of include/exl3_hip.h: argument checks, workspace
// management and dispatch to the gfx950 kernels.  Checks mirror the reference's
// preconditions (src/exl3-ggml.cpp:56-57, src/exl3_codec.cpp:12-19,117-135,
// patches/llama-exl3.patch:81-84,225-235) and turn them into status codes.
#include "exl3_hip.h"
#include "exl3-block.h"

#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <algorithm>
#include <utility>
#include <vector>

#include "exl3_launch.hpp"

namespace {

exl3_status from_hip(hipError_t e) { return e == hipSuccess ? EXL3_OK : EXL3_HIP_ERROR; }

bool valid_rate(unsigned bits, unsigned cb) { return bits >= 1 && bits <= 8 && cb <= 2; }
bool aligned(const void *p, size_t a) { return ((uintptr_t)p % a) == 0; }
bool valid_dtype(exl3_dtype t) { return t == EXL3_F32 || t == EXL3_F16; }
size_t dtype_size(exl3_dtype t) { return t == EXL3_F16 ? 2 : 4; }

constexpr size_t kMaxRows = 65536;
constexpr size_t kMaxDim = (size_t)1 << 24;  // k, n up to 16 Mi (grid and index arithmetic stay in range)

bool valid_matrix(size_t k, size_t n, size_t multiple) {
    return k && n && k % multiple == 0 && n % multiple == 0 && k <= kMaxDim && n <= kMaxDim;
}

// Internal workspaces, one per (device, stream), grown on demand, zero-filled
// when created and kept until process exit.  A workspace that is outgrown is retired, never freed: a call on another thread
// may still be enqueuing kernels that use it.  Growth allocates, so it is
// refused while the stream is being captured into a HIP graph: a caller that
// captures passes its own workspace, or makes one uncaptured call of the
// largest shape first.
struct InternalWs {
    void *ptr = nullptr;
    size_t bytes = 0;
};
std::mutex g_ws_mutex;
std::map<std::pair<int, hipStream_t>, InternalWs> g_ws;
std::vector<void *> g_ws_retired;

exl3_status internal_workspace(size_t need, hipStream_t stream, void **out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return EXL3_HIP_ERROR;
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    InternalWs &ws = g_ws[std::make_pair(dev, stream)];
    if (ws.bytes < need) {
        hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &capture) != hipSuccess) return EXL3_HIP_ERROR;
        if (capture != hipStreamCaptureStatusNone) return EXL3_WORKSPACE_TOO_SMALL;
        const size_t bytes = std::max(need, 2 * ws.bytes);  // geometric growth bounds what is retired
        void *p = nullptr;
        if (hipMalloc(&p, bytes) != hipSuccess) return EXL3_HIP_ERROR;
        if (exl3k::launch_zero(p, bytes, stream) != hipSuccess) {
            (void)hipFree(p);
            return EXL3_HIP_ERROR;
        }
        if (ws.ptr) g_ws_retired.push_back(ws.ptr);
        ws.ptr = p;
        ws.bytes = bytes;
    }
    *out = ws.ptr;
    return EXL3_OK;
}

}  // namespace

extern "C" {

unsigned exl3_hip_version(void) { return EXL3_HIP_VERSION; }

const char *exl3_hip_status_string(exl3_status s) {
    switch (s) {
    case EXL3_OK: return "ok";
    case EXL3_INVAL_PARAMS: return "invalid parameters";
    case EXL3_NO_SUPPORT: return "not supported";
    case EXL3_WORKSPACE_TOO_SMALL: return "workspace too small";
    case EXL3_HIP_ERROR: return "HIP runtime error";
    }
    return "unknown status";
}

size_t exl3_hip_gemv_max_rows(void) { return exl3k::kGemvMaxRows; }

int exl3_hip_supports_mul_mat(unsigned bits, unsigned codebook, size_t k, size_t n, size_t rows, exl3_dtype xt,
                              exl3_dtype yt) {
    return valid_rate(bits, codebook) && valid_matrix(k, n, 128) && rows >= 1 && rows <= kMaxRows &&
           valid_dtype(xt) && valid_dtype(yt);
}

// patches/llama-exl3.patch:69-97: the supports_op rules for ops that touch an
// EXL3 tensor, on plain tensor descriptions; plus the limits of this library's
// kernels (exl3_hip_supports_mul_mat's dimensions, F32/F16 outputs).
static bool is_exl3(const exl3_tensor_info *t) { return t && (t->type >= 43 && t->type <= 45); }
static bool is_2d_groups(const exl3_tensor_info *t) {
    return t->ne[0] > 0 && t->ne[1] > 0 && t->ne[0] % 128 == 0 && t->ne[1] % 128 == 0 && t->ne[2] == 1 &&
           t->ne[3] == 1;
}

int exl3_hip_supports_op(exl3_op op, const exl3_tensor_info *dst, const exl3_tensor_info *src0,
                         const exl3_tensor_info *src1) {
    if (!dst || !src0) return 0;
    switch (op) {
    case EXL3_OP_CPY:
    case EXL3_OP_SET_ROWS:
        if (!is_exl3(dst) && !is_exl3(src0)) return -1;
        return op == EXL3_OP_CPY && src0->type == dst->type && src0->contiguous && dst->contiguous;
    case EXL3_OP_MUL_MAT_ID:
        return is_exl3(src0) ? 0 : -1;
    case EXL3_OP_MUL_MAT: {
        if (!is_exl3(src0)) return -1;
        if (!src1 || !is_2d_groups(src0) || !src0->contiguous) return 0;
        if (src1->type != EXL3_GGML_TYPE_F32 && src1->type != EXL3_GGML_TYPE_F16) return 0;
        if (dst->type != EXL3_GGML_TYPE_F32) return 0;
        const int64_t rows = src1->ne[1] * src1->ne[2] * src1->ne[3];
        if (src1->ne[0] != src0->ne[0] || rows < 1) return 0;
        return exl3_hip_supports_mul_mat(exl3_type_bits(src0->type), EXL3_CB_MUL1, (size_t)src0->ne[0],
                                         (size_t)src0->ne[1], (size_t)rows,
                                         src1->type == EXL3_GGML_TYPE_F16 ? EXL3_F16 : EXL3_F32, EXL3_F32);
    }
    case EXL3_OP_GET_ROWS:
        if (!is_exl3(src0)) return -1;
        if (!src1 || !is_2d_groups(src0) || src1->type != EXL3_GGML_TYPE_I32) return 0;
        if (dst->type != EXL3_GGML_TYPE_F32 && dst->type != EXL3_GGML_TYPE_F16) return 0;
        return exl3_hip_supports_mul_mat(exl3_type_bits(src0->type), EXL3_CB_MUL1, (size_t)src0->ne[0],
                                         (size_t)src0->ne[1], 1, EXL3_F32, EXL3_F32);
    }
    return 0;
}

// The largest plan over every row count 1..rows and both paths a row count can
// take (rows 15..32: the GEMM for one matrix, the GEMV for a group of them), so
// one workspace serves all smaller calls of the same (k, n) in turn (every plan
// starts with the same exchange region).
size_t exl3_hip_mul_mat_workspace_bytes(size_t k, size_t n, size_t rows) {
    if (!valid_matrix(k, n, 128) || rows < 1 || rows > kMaxRows) return 0;
    size_t need = 0;
    const size_t gemv_rows = rows < (size_t)exl3k::kGemvMaxRows ? rows : (size_t)exl3k::kGemvMaxRows;
    for (size_t r = 1; r <= gemv_rows; ++r) {
        const exl3k::GemvPlan p = exl3k::gemv_plan(k, n, r);
        need = std::max(need, p.fits ? p.bytes : exl3k::gemm_plan(k, n, r).bytes);
    }
    // GEMM plans: the largest row count of each (tile height, m-tile count) run;
    // r_hi >= r, so every pass moves on
    for (size_t r = exl3k::kGemvSingleMaxRows + 1; r <= rows;) {
        const int bm = exl3k::gemm_tile_rows(r);
        size_t r_hi = std::min(rows, (r + bm - 1) / bm * bm);
        while (exl3k::gemm_tile_rows(r_hi) != bm) --r_hi;
        need = std::max(need, exl3k::gemm_plan(k, n, r_hi).bytes);
        r = r_hi + 1;
    }
    return need;
}

exl3_status exl3_hip_workspace_init(void *workspace, size_t workspace_bytes, hipStream_t stream) {
    if (!workspace || !aligned(workspace, 256)) return EXL3_INVAL_PARAMS;
    return from_hip(exl3k::launch_zero(workspace, workspace_bytes, stream));
}

static exl3_status mul_mat_impl(const void *records, unsigned bits, unsigned codebook, size_t k, size_t n,
                                const void *x, exl3_dtype xt, size_t rows, size_t x_row_stride, const void *res,
                                size_t res_row_stride, void *y, exl3_dtype yt, size_t y_row_stride, void *workspace,
                                size_t workspace_bytes, hipStream_t stream) {
    if (!exl3_hip_supports_mul_mat(bits, codebook, k, n, rows, xt, yt)) return EXL3_INVAL_PARAMS;
    if (!records || !x || !y || !aligned(records, 16)) return EXL3_INVAL_PARAMS;
    if (!aligned(x, dtype_size(xt)) || !aligned(y, dtype_size(yt))) return EXL3_INVAL_PARAMS;
    if (x_row_stride < k || y_row_stride < n) return EXL3_INVAL_PARAMS;
    const bool gemv = rows <= (size_t)exl3k::kGemvSingleMaxRows && exl3k::gemv_serves(k, n, rows);
    const size_t need = exl3_hip_mul_mat_workspace_bytes(k, n, rows);
    if (workspace) {
        if (!aligned(workspace, 256)) return EXL3_INVAL_PARAMS;
        if (workspace_bytes < need) return EXL3_WORKSPACE_TOO_SMALL;
    } else {
        const exl3_status st = internal_workspace(need, stream, &workspace);
        if (st != EXL3_OK) return st;
    }
    const int xf = xt == EXL3_F16, yf = yt == EXL3_F16;
    if (gemv)
        return from_hip(exl3k::launch_gemv(records, (int)bits, (int)codebook, k, n, x, xf, rows, x_row_stride, y, yf,
                                           y_row_stride, workspace, exl3k::gemv_plan(k, n, rows), stream, res,
                                           res_row_stride));
    return from_hip(exl3k::launch_gemm(records, (int)bits, (int)codebook, k, n, x, xf, rows, x_row_stride, y, yf,
                                       y_row_stride, workspace, exl3k::gemm_plan(k, n, rows), stream, res,
                                       res_row_stride));
}

exl3_status exl3_hip_mul_mat(const void *records, unsigned bits, unsigned codebook, size_t k, size_t n, const void *x,
                             exl3_dtype xt, size_t rows, size_t x_row_stride, void *y, exl3_dtype yt,
                             size_t y_row_stride, void *workspace, size_t workspace_bytes, hipStream_t stream) {
    return mul_mat_impl(records, bits, codebook, k, n, x, xt, rows, x_row_stride, nullptr, 0, y, yt, y_row_stride,
                        workspace, workspace_bytes, stream);
}

exl3_status exl3_hip_mul_mat_add(const void *records, unsigned bits, unsigned codebook, size_t k, size_t n,
                                 const void *x, exl3_dtype xt, size_t rows, size_t x_row_stride, const void *residual,
                                 size_t residual_row_stride, void *y, exl3_dtype yt, size_t y_row_stride,
                                 void *workspace, size_t workspace_bytes, hipStream_t stream) {
    if (!residual || !y || residual_row_stride < n || !aligned(residual, dtype_size(yt))) return EXL3_INVAL_PARAMS;
    if (rows && residual != y) {  // the residual is y itself (same stride) or disjoint from it
        const size_t es = dtype_size(yt);
        const uintptr_t r0 = (uintptr_t)residual, y0 = (uintptr_t)y;
        const uintptr_t r1 = r0 + ((rows - 1) * residual_row_stride + n) * es;
        const uintptr_t y1 = y0 + ((rows - 1) * y_row_stride + n) * es;
        if (r0 < y1 && y0 < r1) return EXL3_INVAL_PARAMS;
    } else if (residual_row_stride != y_row_stride) {
        return EXL3_INVAL_PARAMS;
    }
    return mul_mat_impl(records, bits, codebook, k, n, x, xt, rows, x_row_stride, residual, residual_row_stride, y,
                        yt, y_row_stride, workspace, workspace_bytes, stream);
}

exl3_status exl3_hip_mul_mat_group(const exl3_matrix_desc *mats, size_t count, unsigned bits, unsigned codebook,
                                   size_t k, const void *x, exl3_dtype xt, size_t rows, size_t x_row_stride,
                                   exl3_dtype yt, void *workspace, size_t workspace_bytes, hipStream_t stream) {
    if (!mats || count < 1 || count > (size_t)exl3k::kGemvMaxTargets) return EXL3_INVAL_PARAMS;
    size_t n_total = 0;
    for (size_t i = 0; i < count; ++i) {
        const exl3_matrix_desc &m = mats[i];
        if (!exl3_hip_supports_mul_mat(bits, codebook, k, m.n, rows, xt, yt)) return EXL3_INVAL_PARAMS;
        if (!m.records || !m.y || !aligned(m.records, 16) || !aligned(m.y, dtype_size(yt)) || m.y_row_stride < m.n)
            return EXL3_INVAL_PARAMS;
        n_total += m.n;
    }
    if (!x || !aligned(x, dtype_size(xt)) || x_row_stride < k || n_total > kMaxDim) return EXL3_INVAL_PARAMS;
    // GEMM (or, for one matrix above the single-matrix GEMV rows, whichever
    // exl3_hip_mul_mat picks): one call per matrix, each a full-size launch
    if (!exl3k::gemv_serves(k, n_total, rows) || (count == 1 && rows > (size_t)exl3k::kGemvSingleMaxRows)) {
        for (size_t i = 0; i < count; ++i) {
            const exl3_status st = exl3_hip_mul_mat(mats[i].records, bits, codebook, k, mats[i].n, x, xt, rows,
                                                    x_row_stride, mats[i].y, yt, mats[i].y_row_stride, workspace,
                                                    workspace_bytes, stream);
            if (st != EXL3_OK) return st;
        }
        return EXL3_OK;
    }
    const size_t need = exl3_hip_mul_mat_workspace_bytes(k, n_total, rows);
    if (workspace) {
        if (!aligned(workspace, 256)) return EXL3_INVAL_PARAMS;
        if (workspace_bytes < need) return EXL3_WORKSPACE_TOO_SMALL;
    } else {
        const exl3_status st = internal_workspace(need, stream, &workspace);
        if (st != EXL3_OK) return st;
    }
    exl3k::GemvTargets tg{};
    int nb_end = 0;
    for (size_t i = 0; i < count; ++i) {
        tg.records[i] = (const uint8_t *)mats[i].records;
        tg.y[i] = mats[i].y;
        tg.y_stride[i] = mats[i].y_row_stride;
        nb_end += (int)(mats[i].n / 128);
        tg.nb_end[i] = nb_end;
    }
    tg.count = (int)count;
    return from_hip(exl3k::launch_gemv_targets(tg, (int)bits, (int)codebook, x, xt == EXL3_F16, rows, x_row_stride,
                                               yt == EXL3_F16, workspace, exl3k::gemv_plan(k, n_total, rows), stream));
}

exl3_status exl3_hip_decode_batch(const exl3_decode_desc *descs, size_t count, exl3_layout layout,
                                  unsigned codebook, hipStream_t stream) {
    if (layout != EXL3_LAYOUT_RECORDS && layout != EXL3_LAYOUT_UPSTREAM_TILES) return EXL3_INVAL_PARAMS;
    if (count && !descs) return EXL3_INVAL_PARAMS;
    const size_t mult = layout == EXL3_LAYOUT_RECORDS ? 128 : 16;
    for (size_t i = 0; i < count; ++i) {
        const exl3_decode_desc &d = descs[i];
        if (!valid_rate(d.bits, codebook) || !d.src || !d.out || !aligned(d.src, 16) || !aligned(d.out, 16) ||
            !valid_matrix(d.k, d.n, mult) || (d.k / 16) * ((d.n / 16 + 15) / 16) > (size_t)0x7fffffff)
            return EXL3_INVAL_PARAMS;
    }
    // one launch per (rate, up to kDecodeBatchMax matrices); matrices keep their order within a rate
    const int rl = layout == EXL3_LAYOUT_RECORDS;
    for (unsigned bits = 1; bits <= 8; ++bits) {
        exl3k::DecodeBatch b{};
        size_t wgs = 0;
        auto flush = [&]() -> exl3_status {
            if (!b.count) return EXL3_OK;
            const hipError_t e = exl3k::launch_decode_batch(b, rl, (int)bits, (int)codebook, (unsigned)wgs, stream);
            b = exl3k::DecodeBatch{};
            wgs = 0;
            return from_hip(e);
        };
        for (size_t i = 0; i < count; ++i) {
            const exl3_decode_desc &d = descs[i];
            if (d.bits != bits) continue;
            const size_t mwgs = (d.k / 16) * ((d.n / 16 + 15) / 16);
            if (b.count == exl3k::kDecodeBatchMax || wgs + mwgs > (size_t)0x7fffffff) {
                const exl3_status st = flush();
                if (st != EXL3_OK) return st;
            }
            b.src[b.count] = d.src;
            b.out[b.count] = d.out;
            b.k[b.count] = d.k;
            b.n[b.count] = d.n;
            b.wg_begin[b.count] = (unsigned)wgs;
            ++b.count;
            wgs += mwgs;
        }
        const exl3_status st = flush();
        if (st != EXL3_OK) return st;
    }
    return EXL3_OK;
}

exl3_status exl3_hip_decode(const void *src, exl3_layout layout, unsigned bits, unsigned codebook, size_t k, size_t n,
                            size_t first_column, size_t column_count, uint16_t *out, hipStream_t stream) {
    if (!valid_rate(bits, codebook) || !src || !out || !aligned(src, 16) || !aligned(out, 16)) return EXL3_INVAL_PARAMS;
    const size_t mult = layout == EXL3_LAYOUT_RECORDS ? 128 : 16;
    if (layout != EXL3_LAYOUT_RECORDS && layout != EXL3_LAYOUT_UPSTREAM_TILES) return EXL3_INVAL_PARAMS;
    if (!valid_matrix(k, n, mult)) return EXL3_INVAL_PARAMS;
    if (!column_count || first_column % mult || column_count % mult || first_column > n ||
        column_count > n - first_column)
        return EXL3_INVAL_PARAMS;
    return from_hip(exl3k::launch_decode(src, layout == EXL3_LAYOUT_RECORDS, (int)bits, (int)codebook, k, n,
                                         first_column, column_count, out, stream));
}

exl3_status exl3_hip_reconstruct(const void *src, exl3_layout layout, const uint16_t *su, const uint16_t *sv,
                                 unsigned bits, unsigned codebook, size_t k, size_t n, size_t first_column,
                                 size_t column_count, uint16_t *out, hipStream_t stream) {
    if (!valid_rate(bits, codebook) || !src || !out || !aligned(src, 16) || !aligned(out, 2)) return EXL3_INVAL_PARAMS;
    if (layout != EXL3_LAYOUT_RECORDS && layout != EXL3_LAYOUT_UPSTREAM_TILES) return EXL3_INVAL_PARAMS;
    if (layout == EXL3_LAYOUT_UPSTREAM_TILES && (!su || !sv || !aligned(su, 2) || !aligned(sv, 2)))
        return EXL3_INVAL_PARAMS;
    if (!valid_matrix(k, n, 128)) return EXL3_INVAL_PARAMS;
    if (!column_count || first_column % 128 || column_count % 128 || first_column > n ||
        column_count > n - first_column)
        return EXL3_INVAL_PARAMS;
    return from_hip(exl3k::launch_reconstruct(src, layout == EXL3_LAYOUT_RECORDS, su, sv, (int)bits, (int)codebook, k,
                                              n, first_column, column_count, out, stream));
}

exl3_status exl3_hip_get_rows(const void *records, unsigned bits, unsigned codebook, size_t k, size_t n,
                              const int32_t *ids, size_t count, void *out, exl3_dtype ot, size_t out_row_stride,
                              int *bad_ids, hipStream_t stream) {
    if (!valid_rate(bits, codebook) || !valid_matrix(k, n, 128) || !valid_dtype(ot)) return EXL3_INVAL_PARAMS;
    if (!count) return EXL3_OK;
    if (count > 0x7fffffffu || !records || !ids || !out || !aligned(records, 16) || !aligned(ids, 4) ||
        !aligned(out, dtype_size(ot)) || out_row_stride < k || (bad_ids && !aligned(bad_ids, 4)))
        return EXL3_INVAL_PARAMS;
    return from_hip(exl3k::launch_get_rows(records, (int)bits, (int)codebook, k, n, ids, count, out, ot == EXL3_F16,
                                           out_row_stride, bad_ids, stream));
}

exl3_status exl3_hip_codebook(const uint16_t *states, size_t count, unsigned codebook, uint16_t *out,
                              hipStream_t stream) {
    if (codebook > 2 || (count && (!states || !out))) return EXL3_INVAL_PARAMS;
    if (!count) return EXL3_OK;
    return from_hip(exl3k::launch_codebook(states, count, (int)codebook, out, stream));
}

exl3_status exl3_hip_hadamard128(float *values, size_t count, hipStream_t stream) {
    if (count % 128 || (count && (!values || !aligned(values, 4)))) return EXL3_INVAL_PARAMS;
    return from_hip(exl3k::launch_hadamard(values, count, stream));
}

exl3_status exl3_hip_pack_records(const uint16_t *packed, const uint16_t *su, const uint16_t *sv, unsigned bits,
                                  size_t k, size_t n, void *records, hipStream_t stream) {
    if (bits < 1 || bits > 8 || !valid_matrix(k, n, 128)) return EXL3_INVAL_PARAMS;
    if (!packed || !su || !sv || !records) return EXL3_INVAL_PARAMS;
    if (!aligned(packed, 16) || !aligned(su, 16) || !aligned(sv, 16) || !aligned(records, 16)) return EXL3_INVAL_PARAMS;
    return from_hip(exl3k::launch_pack_records(packed, su, sv, (int)bits, k, n, records, stream));
}

// Workspace of exl3_hip_iface_matmul: the mul_mat workspace (its counters first,
// so one zero-fill covers both), then the packed records.
static size_t iface_records_offset(size_t k, size_t n, size_t batch) {
    return (exl3_hip_mul_mat_workspace_bytes(k, n, batch) + 255) & ~(size_t)255;
}

size_t exl3_hip_iface_matmul_workspace_bytes(unsigned bits, size_t k, size_t n, size_t batch) {
    if (bits < 1 || bits > 8 || !valid_matrix(k, n, 128) || batch < 1 || batch > kMaxRows) return 0;
    return iface_records_offset(k, n, batch) + (n / 128) * (k / 128) * ((size_t)2048 * bits + 512);
}

// exl3_iface_matmul (src/hexagon/exl3_service.c:265-305): the argument checks of
// its first statement (minus the service's memory caps), then the layer.
exl3_status exl3_hip_iface_matmul(unsigned bits, unsigned codebook, size_t k, size_t n, size_t batch,
                                  const uint16_t *packed, const uint16_t *suh, const uint16_t *svh, const float *x,
                                  float *y, void *workspace, size_t workspace_bytes, hipStream_t stream) {
    if (!valid_rate(bits, codebook) || !valid_matrix(k, n, 128) || batch < 1 || batch > kMaxRows)
        return EXL3_INVAL_PARAMS;
    if (!packed || !suh || !svh || !x || !y) return EXL3_INVAL_PARAMS;
    if (!aligned(packed, 16) || !aligned(suh, 16) || !aligned(svh, 16) || !aligned(x, 4) || !aligned(y, 4))
        return EXL3_INVAL_PARAMS;
    const size_t need = exl3_hip_iface_matmul_workspace_bytes(bits, k, n, batch);
    if (workspace) {
        if (!aligned(workspace, 256)) return EXL3_INVAL_PARAMS;
        if (workspace_bytes < need) return EXL3_WORKSPACE_TOO_SMALL;
    } else {
        const exl3_status st = internal_workspace(need, stream, &workspace);
        if (st != EXL3_OK) return st;
    }
    const size_t roff = iface_records_offset(k, n, batch);
    void *records = (uint8_t *)workspace + roff;
    exl3_status st = exl3_hip_pack_records(packed, suh, svh, bits, k, n, records, stream);
    if (st != EXL3_OK) return st;
    return exl3_hip_mul_mat(records, bits, codebook, k, n, x, EXL3_F32, batch, k, y, EXL3_F32, n, workspace, roff,
                            stream);
}

exl3_status exl3_hip_validate_records(const void *records, size_t nbytes, unsigned bits, int *result,
                                      hipStream_t stream) {
    if (bits < 1 || bits > 8 || !result || (nbytes && !records)) return EXL3_INVAL_PARAMS;
    const size_t gb = (size_t)2048 * bits + 512;
    if (nbytes % gb) return EXL3_INVAL_PARAMS;
    return from_hip(exl3k::launch_validate(records, nbytes / gb, (int)bits, result, stream));
}

}  // extern "C"
