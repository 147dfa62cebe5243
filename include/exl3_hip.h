/*
 * exl3_hip.h -- C-ABI of the MI355X (gfx950) EXL3 packed-weight linear layer.
 *
 * Plain pointers and sizes; every pointer named "device" is HIP device memory
 * owned by the caller.  Work is enqueued on the given stream (0 = the null
 * stream) and the functions return without synchronising unless stated.
 * No function throws; every one returns an exl3_status.
 *
 * Reference interfaces replaced (paths are in the reference checkout):
 *   exl3_hip_mul_mat      <- ggml_exl3_mul_mat        src/exl3-ggml.cpp:51-92,
 *                            declared include/exl3-block.h:46, dispatched from
 *                            ggml_compute_forward_mul_mat (patches/llama-exl3.patch:44-51);
 *                            device twin op_exl3_matmul src/exl3-htp.c:159-232
 *   exl3_hip_mul_mat_nd   <- ggml_exl3_mul_mat with its row_offset addressing of
 *                            ggml views (src/exl3-ggml.cpp:11-17, 64, 88)
 *   exl3_hip_get_rows_nd  <- ggml_exl3_get_rows with its id and row addressing
 *                            (src/exl3-ggml.cpp:34-36)
 *   exl3_hip_iface_matmul <- exl3_iface_matmul src/hexagon/exl3_service.c:265-305
 *                            (IDL src/hexagon/exl3_iface.idl:13-15): the same layer on the
 *                            upstream tile layout with separate su / sv, fp32 in and out
 *   exl3_hip_decode       <- exl3::decode_inner(_slice) src/exl3_codec.cpp:123-145
 *                            (and exl3_iface_decode src/hexagon/exl3_iface.idl:5-7)
 *   exl3_hip_reconstruct  <- exl3::reconstruct(_slice)  src/exl3_codec.cpp:169-204
 *   exl3_hip_get_rows     <- ggml_exl3_get_rows        src/exl3-ggml.cpp:19-49,
 *                            declared include/exl3-block.h:47, dispatched from
 *                            ggml_compute_forward_get_rows (patches/llama-exl3.patch:114-121);
 *                            tied embedding exl3::Model::embedding src/exl3_model.cpp:168-187
 *   exl3_hip_codebook     <- exl3::decode_codebook      src/exl3_codec.cpp:68-86
 *   exl3_hip_hadamard128  <- exl3::hadamard128          src/exl3_codec.cpp:147-167
 *   exl3_hip_pack_records <- record assembly tests/test-exl3-graph.cpp:37-45,
 *                            tools/export_native_gguf.py:27-36
 *   exl3_hip_validate_records <- ggml_validate_row_data EXL3 case
 *                            patches/llama-exl3.patch:327-338
 *   exl3_hip_supports_mul_mat <- supports_op predicates patches/llama-exl3.patch:81-84,225-235
 *   exl3_hip_model_*      <- exl3::Model src/exl3_model.cpp:79-187 (include/exl3_model.h),
 *                            for C callers; the C++ class is include/exl3_model.h
 */
#ifndef EXL3_HIP_H
#define EXL3_HIP_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EXL3_HIP_VERSION 10100u /* major * 10000 + minor * 100 + patch */

typedef enum exl3_status {
    EXL3_OK = 0,
    EXL3_INVAL_PARAMS = 1,       /* shape / rate / codebook / stride rejected (HTP_STATUS_INVAL_PARAMS) */
    EXL3_NO_SUPPORT = 2,         /* valid request this build does not implement (HTP_STATUS_NO_SUPPORT) */
    EXL3_WORKSPACE_TOO_SMALL = 3,/* caller workspace below exl3_hip_mul_mat_workspace_bytes() */
    EXL3_HIP_ERROR = 4           /* a HIP runtime call failed (HTP_STATUS_INTERNAL_ERR) */
} exl3_status;

typedef enum exl3_dtype { EXL3_F32 = 0, EXL3_F16 = 1 } exl3_dtype;

/* codebook ids match exl3::Codebook (include/exl3_codec.h) */
typedef enum exl3_codebook { EXL3_CB_3INST = 0, EXL3_CB_MCG = 1, EXL3_CB_MUL1 = 2 } exl3_codebook;

typedef enum exl3_layout {
    EXL3_LAYOUT_UPSTREAM_TILES = 0, /* [k/16][n/16][16*bits] u16, the .trellis tensor */
    EXL3_LAYOUT_RECORDS = 1         /* 128x128 group records, include/exl3-block.h */
} exl3_layout;

unsigned exl3_hip_version(void);
const char *exl3_hip_status_string(exl3_status status);

/* Largest row count served by the register-decode GEMV kernel (32): a grouped
 * call (exl3_hip_mul_mat_group) of at most this many rows is one GEMV launch.
 * exl3_hip_mul_mat runs the GEMV up to 14 rows (16 when a GEMV workgroup's
 * share of k is short: at most 64 (record, row) blocks to prepare) and the
 * LDS-decode MFMA GEMM kernel above, where the GEMM is the faster of the two. */
size_t exl3_hip_gemv_max_rows(void);

/* 1 when exl3_hip_mul_mat accepts this problem: bits 1..8, codebook 0..2,
 * k and n nonzero multiples of 128, 1 <= rows <= 65536, dtypes F32/F16. */
int exl3_hip_supports_mul_mat(unsigned bits, unsigned codebook, size_t k, size_t n, size_t rows,
                              exl3_dtype xt, exl3_dtype yt);

/* ---- engine-side op predicates (ggml supports_op) ------------------------
 * The reference gates the ggml ops that touch an EXL3 tensor in its CPU
 * backend's supports_op (patches/llama-exl3.patch:81-97).  A HIP backend asks
 * exl3_hip_supports_op with the op's tensors described by plain values:
 *   MUL_MAT    src0 EXL3 (types 43/44/45): ne0 and ne1 multiples of 128, ne2 = ne3 = 1,
 *              src0 contiguous, src1 F32 or F16 (patch:81-84); here also dst F32
 *              and the dimensions exl3_hip_mul_mat accepts
 *   MUL_MAT_ID src0 EXL3: unsupported (patch:92-93)
 *   GET_ROWS   src0 EXL3: ne0 and ne1 multiples of 128, ne2 = ne3 = 1, src1 I32
 *              (patch:94-97); here also dst F32 or F16
 *   CPY        dst or src0 EXL3: only a copy between contiguous tensors of the
 *              same EXL3 type, i.e. a byte copy of group records (patch:71-72)
 *   SET_ROWS   dst or src0 EXL3: unsupported (patch:69-72)
 * Returns 1 (served), 0 (refused: keep the op off this backend) or -1 (no EXL3
 * tensor in the op: not this library's decision). */
typedef enum exl3_op {
    EXL3_OP_MUL_MAT = 0,
    EXL3_OP_MUL_MAT_ID = 1,
    EXL3_OP_GET_ROWS = 2,
    EXL3_OP_CPY = 3,
    EXL3_OP_SET_ROWS = 4
} exl3_op;

/* ggml type ids used by the predicates (ggml.h enum ggml_type of the reference's
 * llama.cpp revision; the EXL3 ids are include/exl3-block.h's 43/44/45) */
#define EXL3_GGML_TYPE_F32 0u
#define EXL3_GGML_TYPE_F16 1u
#define EXL3_GGML_TYPE_I32 26u

typedef struct exl3_tensor_info {
    unsigned type;     /* ggml type id */
    int64_t ne[4];     /* ggml ne[]: ne[0] is the row length */
    int contiguous;    /* ggml_is_contiguous() */
    size_t nb[4];      /* ggml nb[]: byte strides of the four dimensions */
} exl3_tensor_info;

/* dst and src0 are required; src1 is required for MUL_MAT, MUL_MAT_ID and GET_ROWS
 * (NULL there: 0).  Beyond the reference's rules, MUL_MAT and GET_ROWS are served
 * when exl3_hip_mul_mat_nd / exl3_hip_get_rows_nd can address every row of the
 * views as the reference's row_offset does (src/exl3-ggml.cpp:11-17):
 *   MUL_MAT   src1 nb[0] = its element size and nb[1..3] multiples of it;
 *             dst F32, ne = [src0 ne[1], src1 ne[1], src1 ne[2], src1 ne[3]],
 *             nb[0] = 4, nb[1..3] multiples of 4, no two dst rows overlapping
 *   GET_ROWS  src1 (ids) ne[3] = 1 and nb[0..2] multiples of 4; dst ne = [src0
 *             ne[0], src1 ne[0], src1 ne[1], src1 ne[2]], nb[0] = its element
 *             size, nb[1..3] multiples of it, no two dst rows overlapping
 * Anything else touching an EXL3 tensor is refused (0), so no view is ever
 * read or written at addresses other than ggml's. */
int exl3_hip_supports_op(exl3_op op, const exl3_tensor_info *dst, const exl3_tensor_info *src0,
                         const exl3_tensor_info *src1);

/* Device workspace bytes exl3_hip_mul_mat needs for (k, n) at any row count
 * 1..rows.  The workspace starts with the 16 MiB of split-K hand-off words,
 * which every call leaves zero, followed by per-call staging: zero-fill it once
 * before its first use (exl3_hip_workspace_init).  One workspace serves any
 * sequence of calls when it holds at least exl3_hip_mul_mat_workspace_bytes(k,
 * n, rows) of every one of them; calls that share one must not run concurrently
 * (order them on one stream).  A GEMV call whose split-K partials would not fit
 * the 16 MiB runs the GEMM path instead (k * n above about 134 M weights at 32
 * rows). */
size_t exl3_hip_mul_mat_workspace_bytes(size_t k, size_t n, size_t rows);
/* Zero-fills workspace_bytes of a caller workspace; NULL: the internal workspace
 * of the current device and this stream, if one exists. */
exl3_status exl3_hip_workspace_init(void *workspace, size_t workspace_bytes, hipStream_t stream);

/* Split-K failure flag of a workspace (NULL: the internal workspace of the current
 * device and this stream).  A GEMV workgroup that sums split partials waits for each
 * other split's words a bounded time (2^20 polls per wave, about a second); one
 * that never arrives gives NaN in the outputs that need it and sets a status word
 * in the workspace.  A partial may then still arrive after the exchange was
 * cleared, so while the word is set every GEMV call with that workspace writes NaN
 * for every output it sums, without waiting; exl3_hip_workspace_init clears it.
 * *faulted = 1 when the word is set, else 0.  Synchronises the stream.  No
 * counterpart in the reference, whose ops run on one thread pool per call. */
exl3_status exl3_hip_workspace_status(const void *workspace, size_t workspace_bytes, int *faulted,
                                      hipStream_t stream);

/* Test hook for the failure path above, never needed by an engine: spin_limit > 0
 * replaces the wait budget (polls per wave) and drop_split >= 0 makes the
 * workgroups of that k split skip storing their partial, so the summing
 * workgroup's own bounded wait runs out and every kernel still ends normally.
 * (0, -1) restores the defaults.  Process-wide; not for concurrent use. */
exl3_status exl3_hip_test_exchange_fault(int spin_limit, int drop_split);

/*
 * y[r][j] = sv[j] * H128( sum_i H128(x[r] * su)[i] * W_hat[i][j] )   (0 <= r < rows)
 * i.e. y = x . diag(su) H W_hat H diag(sv), the EXL3 linear layer, with su taken
 * from record (0, kb) and sv from record (nb, 0) as src/exl3-ggml.cpp:60-90 does.
 *   records      device, (n/128)*(k/128) records of exl3_group_bytes(bits), 16-byte aligned
 *   bits         1..8; codebook 0..2 (the reference's ggml op uses mul1 = 2)
 *   x            device, rows x k of xt, row stride x_row_stride elements (>= k)
 *   y            device, rows x n of yt, row stride y_row_stride elements (>= n)
 *   input range  the kernels hold xh = H128(x[r] * su) / sqrt(128) in fp16 (as a
 *                hi + lo pair up to 16 rows, hi only above), where the reference
 *                keeps fp32: every element of xh must stay below 65520 in
 *                magnitude (true whenever |x[r][i] * su[i]| <= 5790 for all i);
 *                beyond that the affected output rows are Inf or NaN
 *   workspace    device, >= exl3_hip_mul_mat_workspace_bytes(k, n, rows), zero-filled
 *                before first use; NULL -> an internal per-(device, stream)
 *                workspace is allocated on first use and kept (grown, never
 *                freed, when a larger call needs more).  While the stream is
 *                being captured into a HIP graph the internal workspace cannot
 *                grow: such a call returns EXL3_WORKSPACE_TOO_SMALL unless an
 *                uncaptured call of at least this size came first; callers that
 *                capture should pass their own workspace
 * Deterministic: the same inputs give the same bits on every call.
 */
exl3_status exl3_hip_mul_mat(const void *records, unsigned bits, unsigned codebook, size_t k, size_t n,
                             const void *x, exl3_dtype xt, size_t rows, size_t x_row_stride,
                             void *y, exl3_dtype yt, size_t y_row_stride,
                             void *workspace, size_t workspace_bytes, hipStream_t stream);

/* exl3_hip_mul_mat without a workspace and without any allocation: no
 * counterpart in the reference; for callers that cannot allocate (code under
 * HIP-graph capture, serving loops or harnesses that forbid hipMalloc).  The
 * workspace is a 64 MiB device array inside the library, one per GPU, held
 * until the process ends; a call whose exl3_hip_mul_mat_workspace_bytes(k, n,
 * rows) exceeds it returns EXL3_WORKSPACE_TOO_SMALL before anything is
 * enqueued.  Every call on a GPU shares
 * that GPU's array: calls that overlap on one GPU (different streams, or
 * threads without ordering) race and give wrong results; order them on one
 * stream.  Results equal exl3_hip_mul_mat's bit for bit.  A split-K wait that
 * gives up (see exl3_hip_workspace_status) marks the array like any workspace;
 * the array cannot be zero-filled again from outside, so every later call on
 * that GPU that sums split partials writes NaN until the process ends. */
exl3_status exl3_hip_mul_mat_noalloc(const void *records, unsigned bits, unsigned codebook, size_t k, size_t n,
                                     const void *x, exl3_dtype xt, size_t rows, size_t x_row_stride,
                                     void *y, exl3_dtype yt, size_t y_row_stride, hipStream_t stream);

/* y = residual + layer(x): the graph ADD(MUL_MAT(w, x), residual) of
 * tests/test-exl3-graph.cpp:53-55 in one call, the sum formed in fp32 and
 * rounded once to yt.  residual: device, rows x n of yt, row stride
 * residual_row_stride (>= n); it is either y itself with y's stride (an in-place
 * accumulate) or disjoint from y.  Otherwise as exl3_hip_mul_mat.  The
 * reference declines this fusion for its kernels (patches/llama-exl3.patch:161-162)
 * and runs the ADD as a separate graph node. */
exl3_status exl3_hip_mul_mat_add(const void *records, unsigned bits, unsigned codebook, size_t k, size_t n,
                                 const void *x, exl3_dtype xt, size_t rows, size_t x_row_stride,
                                 const void *residual, size_t residual_row_stride,
                                 void *y, exl3_dtype yt, size_t y_row_stride,
                                 void *workspace, size_t workspace_bytes, hipStream_t stream);

/* One matrix of an exl3_hip_mul_mat_group call. */
typedef struct exl3_matrix_desc {
    const void *records;   /* device, (n/128)*(k/128) group records, 16-byte aligned */
    size_t n;              /* output features, multiple of 128 */
    void *y;               /* device, rows x n of the call's yt */
    size_t y_row_stride;   /* elements, >= n */
} exl3_matrix_desc;

/* y_i = layer_i(x) for 1..4 matrices that share k, bits, codebook, x and rows
 * (the q/k/v or gate/up projections of one decoder layer): at rows <=
 * exl3_hip_gemv_max_rows() one GEMV launch serves all of them, so the launch and
 * its latency chain are paid once; larger row counts run one exl3_hip_mul_mat
 * per matrix.  Each y_i is the exl3_hip_mul_mat result within the layer
 * tolerance (the split of k follows the total width, so the summation order may
 * differ from a single call's).  workspace: >= exl3_hip_mul_mat_workspace_bytes(k,
 * sum of n_i, rows), or NULL for the internal one.  This entry point has no
 * counterpart in the reference, whose ggml op multiplies one matrix per call. */
exl3_status exl3_hip_mul_mat_group(const exl3_matrix_desc *mats, size_t count, unsigned bits, unsigned codebook,
                                   size_t k, const void *x, exl3_dtype xt, size_t rows, size_t x_row_stride,
                                   exl3_dtype yt, void *workspace, size_t workspace_bytes, hipStream_t stream);

/* Workspace bytes of an exl3_hip_mul_mat_group call: the most any row count
 * 1..rows needs, whether the call runs as one GEMV launch over the total width or
 * as one exl3_hip_mul_mat per matrix (a narrower matrix may need more split
 * partials than the total width does).  0 for invalid arguments. */
size_t exl3_hip_mul_mat_group_workspace_bytes(size_t k, const size_t *n, size_t count, size_t rows);

/* The ggml op on ggml views, replacing ggml_exl3_mul_mat (src/exl3-ggml.cpp:51-92)
 * with its row addressing: row r = i1 + ne[1] (i2 + ne[2] i3) of x starts at byte
 * i1 nb[1] + i2 nb[2] + i3 nb[3] of x, and its output row at the same indices of y
 * (row_offset, src/exl3-ggml.cpp:11-17, used at :64 and :88).
 *   x_info  type EXL3_GGML_TYPE_F32 or _F16, ne[0] = k, nb[0] = its element size,
 *           nb[1..3] multiples of it, in any order (permuted and sliced views)
 *   y_info  type F32 or F16, ne[0] = n, ne[1..3] = x's, nb[0] = its element size,
 *           nb[1..3] multiples of it, no two rows overlapping
 *   (the contiguous fields are not read)
 * The longest run of row dimensions that both views step through with one
 * stride is one exl3_hip_mul_mat call; the other dimensions loop over such calls.
 * workspace: >= exl3_hip_mul_mat_workspace_bytes(k, n, ne[1] ne[2] ne[3]), or NULL.
 * Each row is within exl3_hip_mul_mat's tolerance (which kernel serves a row
 * depends on how many rows share its call). */
exl3_status exl3_hip_mul_mat_nd(const void *records, unsigned bits, unsigned codebook, size_t k, size_t n,
                                const void *x, const exl3_tensor_info *x_info, void *y,
                                const exl3_tensor_info *y_info, void *workspace, size_t workspace_bytes,
                                hipStream_t stream);

/* Decode packed weights to row-major fp16 bits out[k][column_count] for
 * columns [first_column, first_column + column_count), bit-exact with
 * exl3::decode_inner_slice.  UPSTREAM_TILES: k, n, first and count multiples
 * of 16; RECORDS: multiples of 128.  out is device memory. */
exl3_status exl3_hip_decode(const void *src, exl3_layout layout, unsigned bits, unsigned codebook,
                            size_t k, size_t n, size_t first_column, size_t column_count,
                            uint16_t *out, hipStream_t stream);

/* One matrix of an exl3_hip_decode_batch call. */
typedef struct exl3_decode_desc {
    const void *src;   /* device, packed weights in the call's layout, 16-byte aligned */
    size_t k, n;       /* shape (multiples of 16 for UPSTREAM_TILES, of 128 for RECORDS) */
    uint16_t *out;     /* device, row-major fp16 bits out[k][n], 16-byte aligned */
    unsigned bits;     /* 1..8 */
} exl3_decode_desc;

/* exl3_hip_decode of whole matrices, many per launch: the matrices of one rate
 * share a launch (up to 32 each), so a model's weight set decodes in a few
 * launches instead of one per tensor; output bit-identical to exl3_hip_decode.
 * count 0 is a no-op.  This entry point has no counterpart in the reference,
 * which decodes one tensor per decode_inner call (src/exl3_codec.cpp:117-145). */
exl3_status exl3_hip_decode_batch(const exl3_decode_desc *descs, size_t count, exl3_layout layout,
                                  unsigned codebook, hipStream_t stream);

/* Original-basis weights diag(su) H W_hat H diag(sv) as fp16 bits out[k][column_count],
 * bit-exact with exl3::reconstruct_slice.  UPSTREAM_TILES takes su (k) and sv (n)
 * fp16 device vectors; RECORDS reads them from the records (su/sv may be NULL).
 * k, n, first_column, column_count multiples of 128. */
exl3_status exl3_hip_reconstruct(const void *src, exl3_layout layout, const uint16_t *su,
                                 const uint16_t *sv, unsigned bits, unsigned codebook, size_t k,
                                 size_t n, size_t first_column, size_t column_count, uint16_t *out,
                                 hipStream_t stream);

/* GET_ROWS: out[r][0..k) = column ids[r] of the original-basis weight
 * diag(su) H W_hat H diag(sv), i.e. for every kb the reconstruct of record
 * (ids[r] / 128, kb) as a 128x128 matrix (exl3::reconstruct, fp16-rounded),
 * column ids[r] % 128; bit-exact, widened to fp32 for ot = F32 (ggml's dst type).
 *   records        device, as exl3_hip_mul_mat; codebook: the reference uses mul1 = 2
 *   ids            device int32[count] (GGML_TYPE_I32 ids)
 *   out            device, count rows of ot, row stride out_row_stride (>= k) elements
 *   bad_ids        optional device int: set to 1 when some id is outside [0, n)
 *                  (its row is NaN); the reference asserts instead
 * count == 0 is a no-op. */
exl3_status exl3_hip_get_rows(const void *records, unsigned bits, unsigned codebook, size_t k, size_t n,
                              const int32_t *ids, size_t count, void *out, exl3_dtype ot, size_t out_row_stride,
                              int *bad_ids, hipStream_t stream);

/* GET_ROWS on ggml views (ggml_exl3_get_rows, src/exl3-ggml.cpp:19-49): id
 * r = i0 + ne[0] (i1 + ne[1] i2) is read at byte i0 nb[0] + i1 nb[1] + i2 nb[2] of
 * ids, and its row written at byte i0 nb[1] + i1 nb[2] + i2 nb[3] of out (:34-36).
 *   ids_info  type EXL3_GGML_TYPE_I32, ne[3] = 1, nb[0..2] multiples of 4
 *   out_info  type F32 or F16, ne = [k, ids ne[0], ids ne[1], ids ne[2]], nb[0] =
 *             its element size, nb[1..3] multiples of it, no two rows overlapping
 * Otherwise as exl3_hip_get_rows; no ids (a zero ne) is a no-op. */
exl3_status exl3_hip_get_rows_nd(const void *records, unsigned bits, unsigned codebook, size_t k, size_t n,
                                 const int32_t *ids, const exl3_tensor_info *ids_info, void *out,
                                 const exl3_tensor_info *out_info, int *bad_ids, hipStream_t stream);

/* out[i] = fp16 codebook value of states[i], bit-exact with exl3::decode_codebook. */
exl3_status exl3_hip_codebook(const uint16_t *states, size_t count, unsigned codebook, uint16_t *out,
                              hipStream_t stream);

/* In-place orthonormal H128 over each consecutive 128 fp32 values (count % 128 == 0),
 * bit-exact with exl3::hadamard128. */
exl3_status exl3_hip_hadamard128(float *values, size_t count, hipStream_t stream);

/* Upstream tiles [k/16][n/16][16*bits] + su[k] + sv[n] -> records. */
exl3_status exl3_hip_pack_records(const uint16_t *packed, const uint16_t *su, const uint16_t *sv,
                                  unsigned bits, size_t k, size_t n, void *records, hipStream_t stream);

/* The DSP service's layer exl3_iface_matmul (src/hexagon/exl3_service.c:265-305,
 * IDL src/hexagon/exl3_iface.idl:13-15): y = x . diag(su) H W_hat H diag(sv) on the
 * upstream tile layout with separate su / sv vectors, fp32 in and out.  One call packs
 * the tiles and scales into group records inside the workspace (exl3_hip_pack_records)
 * and runs exl3_hip_mul_mat on them, so the weights are decoded once per call, as the
 * service decodes them; callers that reuse the weights pack once and call
 * exl3_hip_mul_mat instead.
 *   packed      device, [k/16][n/16][16*bits] u16 = k*n*bits/8 bytes, 16-byte aligned
 *   suh, svh    device fp16 su[k] and sv[n], 16-byte aligned
 *   x, y        device fp32, batch x k and batch x n, dense rows (the service's layout)
 *   workspace   >= exl3_hip_iface_matmul_workspace_bytes(bits, k, n, batch), 256-byte
 *               aligned, zero-filled before first use; NULL -> an internal one
 * The service also caps batch at 8 and k*n at 64 Mi (its memory); here batch is any row
 * count exl3_hip_mul_mat accepts.  Rejections follow the service: bits 1..8, codebook
 * 0..2, k and n nonzero multiples of 128, batch >= 1 (EXL3_INVAL_PARAMS where the
 * service returns 2). */
size_t exl3_hip_iface_matmul_workspace_bytes(unsigned bits, size_t k, size_t n, size_t batch);
exl3_status exl3_hip_iface_matmul(unsigned bits, unsigned codebook, size_t k, size_t n, size_t batch,
                                  const uint16_t *packed, const uint16_t *suh, const uint16_t *svh, const float *x,
                                  float *y, void *workspace, size_t workspace_bytes, hipStream_t stream);

/* *result (device int) = 1 when every su/sv value of every record is finite,
 * 0 otherwise; EXL3_INVAL_PARAMS when nbytes is not a whole number of records. */
exl3_status exl3_hip_validate_records(const void *records, size_t nbytes, unsigned bits, int *result,
                                      hipStream_t stream);

/* ---- deployment model reader (exl3::Model, src/exl3_model.cpp:79-187) ----
 * A model directory holds model.safetensors and hexagon-exl3.json; it is
 * validated as the reference validates it.  Host memory maps the file; the
 * embedding and the record upload use the current HIP device. */
typedef struct exl3_model exl3_model;

/* NULL when the directory is missing or malformed; the reason is copied into
 * error (NUL-terminated, at most error_bytes - 1 characters) when given. */
exl3_model *exl3_hip_model_open(const char *directory, char *error, size_t error_bytes);
void exl3_hip_model_close(exl3_model *model);
size_t exl3_hip_model_tensor_count(const exl3_model *model);
size_t exl3_hip_model_payload_bytes(const exl3_model *model);
size_t exl3_hip_model_hidden_size(const exl3_model *model);
size_t exl3_hip_model_vocab_size(const exl3_model *model);
double exl3_hip_model_bits_per_weight(const exl3_model *model);
/* out (host) = hidden_size fp16 bits of token's tied embedding, bit-exact with
 * exl3::Model::embedding; EXL3_INVAL_PARAMS when token >= vocab_size. */
exl3_status exl3_hip_model_embedding(const exl3_model *model, uint32_t token, uint16_t *out);
/* EXL3 matrices of the model (every <prefix>.trellis with its .suh/.svh), in name order */
size_t exl3_hip_model_matrix_count(const exl3_model *model);
exl3_status exl3_hip_model_matrix(const exl3_model *model, size_t index, char *name, size_t name_bytes,
                                  unsigned *bits, unsigned *codebook, size_t *k, size_t *n);
/* device bytes of matrix index's group records (0 for a bad index) */
size_t exl3_hip_model_record_bytes(const exl3_model *model, size_t index);
/* Row-coded EXL3 embedding tables of the model: every <prefix>.trellis of rank 2
 * (I16 [rows, groups * words]) that has a <prefix>.signs (F16 [groups, 256]),
 * validated as the reference's model audit validates them
 * (tools/inspect_model.py:78-90): words = 16 * bits + 1 per group, bits 1..8.
 * Their decode is not implemented (the reference's runtime has none either).
 * EXL3_OK with *count, or EXL3_INVAL_PARAMS with the audit's reason copied into
 * error ("Invalid EXL3 embedding: <name>", "... groups: ...", "... bitrate: ..."). */
exl3_status exl3_hip_model_embedding_tables(const exl3_model *model, size_t *count, char *error, size_t error_bytes);
/* table index (name order): its prefix, rows, groups, bits and padded width
 * (groups * 256) */
exl3_status exl3_hip_model_embedding_table(const exl3_model *model, size_t index, char *name, size_t name_bytes,
                                           size_t *rows, size_t *groups, unsigned *bits, size_t *width_padded);
/* packs matrix index into group records at device pointer records (16-byte
 * aligned, exl3_hip_model_record_bytes long), ready for exl3_hip_mul_mat;
 * returns when they are complete.  k and n must be multiples of 128. */
exl3_status exl3_hip_model_upload_records(const exl3_model *model, size_t index, void *records, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* EXL3_HIP_H */
