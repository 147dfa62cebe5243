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
// kernels (exl3_hip_supports_mul_mat's dimensions, F32/F16 outputs) and the
// views exl3_hip_mul_mat_nd / exl3_hip_get_rows_nd can address.
static bool is_exl3(const exl3_tensor_info *t) { return t && (t->type >= 43 && t->type <= 45); }
static bool is_2d_groups(const exl3_tensor_info *t) {
    return t->ne[0] > 0 && t->ne[1] > 0 && t->ne[0] % 128 == 0 && t->ne[1] % 128 == 0 && t->ne[2] == 1 &&
           t->ne[3] == 1;
}

// A ggml view as rows (src/exl3-ggml.cpp:11-17): row r = i1 + ne[1] (i2 + ne[2] i3)
// starts at byte i1 nb[1] + i2 nb[2] + i3 nb[3].  Valid when dimension 0 is dense
// (nb[0] = es), every row stride is a multiple of es, and the row count is in
// range; with `disjoint` no two rows may share a byte (the view is written).
static bool rows_view_ok(const exl3_tensor_info *t, size_t es, int64_t row_len, bool disjoint) {
    if (t->ne[0] != row_len || t->nb[0] != es) return false;
    size_t rows = 1;
    for (int d = 1; d < 4; ++d) {
        if (t->ne[d] < 0 || (size_t)t->ne[d] > kMaxRows || t->nb[d] % es) return false;
        rows *= (size_t)t->ne[d];
        if (rows > kMaxRows) return false;
    }
    if (!disjoint) return true;
    // the dimensions that step (ne > 1) in stride order: each stride must clear
    // the extent of the rows below it (a sufficient condition for no overlap)
    std::pair<size_t, size_t> dims[3];
    int c = 0;
    for (int d = 1; d < 4; ++d)
        if (t->ne[d] > 1) dims[c++] = std::make_pair(t->nb[d], (size_t)t->ne[d]);
    std::sort(dims, dims + c);
    size_t extent = (size_t)row_len * es;
    for (int i = 0; i < c; ++i) {
        if (dims[i].first < extent) return false;
        if (dims[i].first > SIZE_MAX / dims[i].second) return false;  // an address range no device has
        extent = dims[i].first * dims[i].second;
    }
    return true;
}
static size_t view_rows(const exl3_tensor_info *t) { return (size_t)t->ne[1] * (size_t)t->ne[2] * (size_t)t->ne[3]; }
static bool dtype_of(unsigned ggml_type, exl3_dtype *dt) {
    if (ggml_type == EXL3_GGML_TYPE_F32) *dt = EXL3_F32;
    else if (ggml_type == EXL3_GGML_TYPE_F16) *dt = EXL3_F16;
    else return false;
    return true;
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
        exl3_dtype xt;
        if (!dtype_of(src1->type, &xt) || dst->type != EXL3_GGML_TYPE_F32) return 0;
        // dst = [ne01, ne11, ne12, ne13]; every row of src1 and dst addressable
        if (dst->ne[0] != src0->ne[1] || dst->ne[1] != src1->ne[1] || dst->ne[2] != src1->ne[2] ||
            dst->ne[3] != src1->ne[3])
            return 0;
        if (!rows_view_ok(src1, dtype_size(xt), src0->ne[0], false) || !rows_view_ok(dst, 4, src0->ne[1], true))
            return 0;
        return exl3_hip_supports_mul_mat(exl3_type_bits(src0->type), EXL3_CB_MUL1, (size_t)src0->ne[0],
                                         (size_t)src0->ne[1], view_rows(src1), xt, EXL3_F32);
    }
    case EXL3_OP_GET_ROWS: {
        if (!is_exl3(src0)) return -1;
        if (!src1 || !is_2d_groups(src0) || !src0->contiguous || src1->type != EXL3_GGML_TYPE_I32) return 0;
        exl3_dtype ot;
        if (!dtype_of(dst->type, &ot)) return 0;
        // ids [ne10, ne11, ne12] (ne13 = 1) -> dst [ne00, ne10, ne11, ne12]
        if (src1->ne[3] != 1 || src1->nb[0] % 4 || src1->nb[1] % 4 || src1->nb[2] % 4) return 0;
        if (dst->ne[0] != src0->ne[0] || dst->ne[1] != src1->ne[0] || dst->ne[2] != src1->ne[1] ||
            dst->ne[3] != src1->ne[2])
            return 0;
        if (!rows_view_ok(dst, dtype_size(ot), src0->ne[0], true)) return 0;
        return exl3_hip_supports_mul_mat(exl3_type_bits(src0->type), EXL3_CB_MUL1, (size_t)src0->ne[0],
                                         (size_t)src0->ne[1], 1, EXL3_F32, EXL3_F32);
    }
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
    if (!workspace) {  // the internal workspace of (current device, stream), if there is one
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) return EXL3_HIP_ERROR;
        std::lock_guard<std::mutex> lock(g_ws_mutex);
        const auto it = g_ws.find(std::make_pair(dev, stream));
        if (it == g_ws.end() || !it->second.ptr) return EXL3_OK;
        return from_hip(exl3k::launch_zero(it->second.ptr, it->second.bytes, stream));
    }
    if (!aligned(workspace, 256)) return EXL3_INVAL_PARAMS;
    return from_hip(exl3k::launch_zero(workspace, workspace_bytes, stream));
}

exl3_status exl3_hip_workspace_status(const void *workspace, size_t workspace_bytes, int *faulted,
                                      hipStream_t stream) {
    if (!faulted) return EXL3_INVAL_PARAMS;
    *faulted = 0;
    const uint8_t *ws = (const uint8_t *)workspace;
    if (!ws) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) return EXL3_HIP_ERROR;
        std::lock_guard<std::mutex> lock(g_ws_mutex);
        const auto it = g_ws.find(std::make_pair(dev, stream));
        if (it == g_ws.end() || !it->second.ptr) return EXL3_OK;  // never used: nothing can have failed
        ws = (const uint8_t *)it->second.ptr;
    } else if (!aligned(ws, 256) || workspace_bytes < exl3k::kSharedPrefixBytes) {
        return EXL3_INVAL_PARAMS;
    }
    uint32_t word = 0;
    if (hipMemcpyAsync(&word, ws + exl3k::kStatusOffset, sizeof(word), hipMemcpyDeviceToHost, stream) != hipSuccess ||
        hipStreamSynchronize(stream) != hipSuccess)
        return EXL3_HIP_ERROR;
    *faulted = word != 0u;
    return EXL3_OK;
}

exl3_status exl3_hip_test_exchange_fault(int spin_limit, int drop_split) {
    exl3k::set_exchange_fault(spin_limit, drop_split);
    return EXL3_OK;
}

static exl3_status mul_mat_impl(const void *records, unsigned bits, unsigned codebook, size_t k, size_t n,
                                const void *x, exl3_dtype xt, size_t rows, size_t x_row_stride, const void *res,
                                size_t res_row_stride, void *y, exl3_dtype yt, size_t y_row_stride, void *workspace,
                                size_t workspace_bytes, hipStream_t stream) {
    if (!exl3_hip_supports_mul_mat(bits, codebook, k, n, rows, xt, yt)) return EXL3_INVAL_PARAMS;
    if (!records || !x || !y || !aligned(records, 16)) return EXL3_INVAL_PARAMS;
    if (!aligned(x, dtype_size(xt)) || !aligned(y, dtype_size(yt))) return EXL3_INVAL_PARAMS;
    if (x_row_stride < k || y_row_stride < n) return EXL3_INVAL_PARAMS;
    const bool gemv = exl3k::gemv_serves_single(k, n, rows);
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
    // the workspace is checked (or the internal one grown) before anything is
    // enqueued, for whichever of the two paths below the call takes
    size_t ns[exl3k::kGemvMaxTargets];
    for (size_t i = 0; i < count; ++i) ns[i] = mats[i].n;
    const size_t need = exl3_hip_mul_mat_group_workspace_bytes(k, ns, count, rows);
    if (workspace) {
        if (!aligned(workspace, 256)) return EXL3_INVAL_PARAMS;
        if (workspace_bytes < need) return EXL3_WORKSPACE_TOO_SMALL;
    } else {
        const exl3_status st = internal_workspace(need, stream, &workspace);
        if (st != EXL3_OK) return st;
        workspace_bytes = need;
    }
    // GEMM (or, for one matrix above the single-matrix GEMV rows, whichever
    // exl3_hip_mul_mat picks): one call per matrix, each a full-size launch
    if (!exl3k::gemv_serves(k, n_total, rows) || (count == 1 && !exl3k::gemv_serves_single(k, n_total, rows))) {
        for (size_t i = 0; i < count; ++i) {
            const exl3_status st = exl3_hip_mul_mat(mats[i].records, bits, codebook, k, mats[i].n, x, xt, rows,
                                                    x_row_stride, mats[i].y, yt, mats[i].y_row_stride, workspace,
                                                    workspace_bytes, stream);
            if (st != EXL3_OK) return st;
        }
        return EXL3_OK;
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

size_t exl3_hip_mul_mat_group_workspace_bytes(size_t k, const size_t *n, size_t count, size_t rows) {
    if (!n || count < 1 || count > (size_t)exl3k::kGemvMaxTargets) return 0;
    size_t n_total = 0, need = 0;
    for (size_t i = 0; i < count; ++i) {
        const size_t b = exl3_hip_mul_mat_workspace_bytes(k, n[i], rows);
        if (!b) return 0;
        need = std::max(need, b);  // the per-matrix calls of the GEMM path
        n_total += n[i];
    }
    if (n_total > kMaxDim) return 0;
    return std::max(need, exl3_hip_mul_mat_workspace_bytes(k, n_total, rows));  // the one GEMV launch
}

exl3_status exl3_hip_mul_mat_nd(const void *records, unsigned bits, unsigned codebook, size_t k, size_t n,
                                const void *x, const exl3_tensor_info *x_info, void *y,
                                const exl3_tensor_info *y_info, void *workspace, size_t workspace_bytes,
                                hipStream_t stream) {
    exl3_dtype xt, yt;
    if (!x_info || !y_info || !dtype_of(x_info->type, &xt) || !dtype_of(y_info->type, &yt)) return EXL3_INVAL_PARAMS;
    const size_t xes = dtype_size(xt), yes = dtype_size(yt);
    if (!valid_matrix(k, n, 128)) return EXL3_INVAL_PARAMS;
    if (!rows_view_ok(x_info, xes, (int64_t)k, false) || !rows_view_ok(y_info, yes, (int64_t)n, true))
        return EXL3_INVAL_PARAMS;
    for (int d = 1; d < 4; ++d)
        if (x_info->ne[d] != y_info->ne[d]) return EXL3_INVAL_PARAMS;
    const size_t rows = view_rows(x_info);
    if (!exl3_hip_supports_mul_mat(bits, codebook, k, n, rows, xt, yt) || !records || !x || !y)
        return EXL3_INVAL_PARAMS;
    const size_t need = exl3_hip_mul_mat_workspace_bytes(k, n, rows);  // every call below needs at most this
    if (workspace) {
        if (!aligned(workspace, 256)) return EXL3_INVAL_PARAMS;
        if (workspace_bytes < need) return EXL3_WORKSPACE_TOO_SMALL;
    } else {
        const exl3_status st = internal_workspace(need, stream, &workspace);
        if (st != EXL3_OK) return st;
        workspace_bytes = need;
    }
    // Row dimensions 1, 2, 3 in order join one run while both views step through
    // them with one row stride (a run's stride at least a row, as exl3_hip_mul_mat
    // takes it); the run is one call, the dimensions from `outer` on loop.
    size_t run = 1, xs = k, ys = n;  // rows of the run, its strides in elements
    int outer = 4;
    for (int d = 1; d < 4 && outer == 4; ++d) {
        const size_t ne = (size_t)x_info->ne[d], xnb = x_info->nb[d] / xes, ynb = y_info->nb[d] / yes;
        if (ne == 1) continue;
        if (run == 1 && xnb >= k && ynb >= n) {
            xs = xnb;
            ys = ynb;
            run = ne;
        } else if (run > 1 && xnb == xs * run && ynb == ys * run) {
            run *= ne;
        } else {
            outer = d;
        }
    }
    size_t count[4] = {1, 1, 1, 1};
    for (int d = outer; d < 4; ++d) count[d] = (size_t)x_info->ne[d];
    for (size_t i3 = 0; i3 < count[3]; ++i3)
        for (size_t i2 = 0; i2 < count[2]; ++i2)
            for (size_t i1 = 0; i1 < count[1]; ++i1) {
                const size_t xo = i1 * x_info->nb[1] + i2 * x_info->nb[2] + i3 * x_info->nb[3];
                const size_t yo = i1 * y_info->nb[1] + i2 * y_info->nb[2] + i3 * y_info->nb[3];
                const exl3_status st = mul_mat_impl(records, bits, codebook, k, n, (const uint8_t *)x + xo, xt, run,
                                                    xs, nullptr, 0, (uint8_t *)y + yo, yt, ys, workspace,
                                                    workspace_bytes, stream);
                if (st != EXL3_OK) return st;
            }
    return EXL3_OK;
}

exl3_status exl3_hip_get_rows_nd(const void *records, unsigned bits, unsigned codebook, size_t k, size_t n,
                                 const int32_t *ids, const exl3_tensor_info *ids_info, void *out,
                                 const exl3_tensor_info *out_info, int *bad_ids, hipStream_t stream) {
    exl3_dtype ot;
    if (!ids_info || !out_info || !dtype_of(out_info->type, &ot)) return EXL3_INVAL_PARAMS;
    if (!valid_rate(bits, codebook) || !valid_matrix(k, n, 128)) return EXL3_INVAL_PARAMS;
    if (ids_info->type != EXL3_GGML_TYPE_I32 || ids_info->ne[3] != 1) return EXL3_INVAL_PARAMS;
    for (int d = 0; d < 3; ++d)
        if (ids_info->ne[d] < 0 || ids_info->nb[d] % 4 || out_info->ne[d + 1] != ids_info->ne[d])
            return EXL3_INVAL_PARAMS;
    const size_t es = dtype_size(ot);
    if (!rows_view_ok(out_info, es, (int64_t)k, true)) return EXL3_INVAL_PARAMS;
    const size_t per = (size_t)ids_info->ne[0];
    if (!view_rows(out_info)) return EXL3_OK;
    if (!records || !ids || !out || !aligned(records, 16) || !aligned(ids, 4) || !aligned(out, es) ||
        (bad_ids && !aligned(bad_ids, 4)))
        return EXL3_INVAL_PARAMS;
    // one launch per (i1, i2) of the ids: ne[0] ids at stride nb[0], their rows at
    // stride out nb[1] (any stride serves a single row)
    const size_t out_stride = per > 1 ? out_info->nb[1] / es : k;
    for (int64_t i2 = 0; i2 < ids_info->ne[2]; ++i2)
        for (int64_t i1 = 0; i1 < ids_info->ne[1]; ++i1) {
            const int32_t *id = (const int32_t *)((const uint8_t *)ids + i1 * ids_info->nb[1] + i2 * ids_info->nb[2]);
            void *o = (uint8_t *)out + i1 * out_info->nb[2] + i2 * out_info->nb[3];
            const hipError_t e = exl3k::launch_get_rows(records, (int)bits, (int)codebook, k, n, id,
                                                        ids_info->nb[0] / 4, per, o, ot == EXL3_F16, out_stride,
                                                        bad_ids, stream);
            if (e != hipSuccess) return EXL3_HIP_ERROR;
        }
    return EXL3_OK;
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
            const size_t mwgs = ((d.k / 16) * ((d.n / 16 + 15) / 16) + exl3k::kDecodeBlocksPerWg - 1) / exl3k::kDecodeBlocksPerWg;
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
    return from_hip(exl3k::launch_get_rows(records, (int)bits, (int)codebook, k, n, ids, 1, count, out, ot == EXL3_F16,
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
