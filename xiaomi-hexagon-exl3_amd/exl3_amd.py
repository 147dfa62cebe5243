"""ctypes binding of the EXL3 HIP C-ABI (include/exl3_hip.h) for Python callers.

Device buffers are torch tensors on a HIP device (torch is used for device
memory and streams only).  Every call goes to libexl3_hip.so; if the library
is missing the import fails -- there is no CPU fallback.
"""
import ctypes
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libexl3_hip.so"

OK, INVAL_PARAMS, NO_SUPPORT, WORKSPACE_TOO_SMALL, HIP_ERROR = range(5)
F32, F16 = 0, 1
CB_3INST, CB_MCG, CB_MUL1 = 0, 1, 2
LAYOUT_UPSTREAM_TILES, LAYOUT_RECORDS = 0, 1

EXPORTS = [
    "exl3_hip_version", "exl3_hip_status_string", "exl3_hip_gemv_max_rows", "exl3_hip_supports_mul_mat",
    "exl3_hip_mul_mat_workspace_bytes", "exl3_hip_workspace_init", "exl3_hip_mul_mat", "exl3_hip_decode",
    "exl3_hip_reconstruct", "exl3_hip_get_rows", "exl3_hip_codebook", "exl3_hip_hadamard128",
    "exl3_hip_pack_records", "exl3_hip_validate_records",
    "exl3_hip_mul_mat_group", "exl3_hip_mul_mat_add", "exl3_hip_decode_batch",
    "exl3_hip_model_open", "exl3_hip_model_close", "exl3_hip_model_tensor_count", "exl3_hip_model_payload_bytes",
    "exl3_hip_model_hidden_size", "exl3_hip_model_vocab_size", "exl3_hip_model_bits_per_weight",
    "exl3_hip_model_embedding", "exl3_hip_model_matrix_count", "exl3_hip_model_matrix", "exl3_hip_model_record_bytes",
    "exl3_hip_model_upload_records", "exl3_hip_iface_matmul_workspace_bytes", "exl3_hip_iface_matmul",
    "exl3_hip_supports_op", "exl3_hip_model_embedding_tables", "exl3_hip_model_embedding_table",
    "exl3_hip_mul_mat_noalloc", "exl3_hip_mul_mat_nd", "exl3_hip_get_rows_nd",
    "exl3_hip_mul_mat_group_workspace_bytes", "exl3_hip_workspace_status", "exl3_hip_test_exchange_fault",
]

# ggml op predicates (exl3_hip_supports_op)
OP_MUL_MAT, OP_MUL_MAT_ID, OP_GET_ROWS, OP_CPY, OP_SET_ROWS = range(5)
GGML_F32, GGML_F16, GGML_I32 = 0, 1, 26


# bytes per ggml block and elements per block of the types used here (ggml's type
# traits; the EXL3 types 43/44/45 are 128-element blocks of 16 K + 4 bytes)
GGML_TYPE_BLOCK = {0: (4, 1), 1: (2, 1), 26: (4, 1), 27: (8, 1), 30: (2, 1),
                   43: (68, 128), 44: (100, 128), 45: (132, 128)}


class TensorInfo(ctypes.Structure):
    """exl3_tensor_info: a ggml tensor's type, ne[4], contiguity and nb[4] (byte strides)"""
    _fields_ = [("type", ctypes.c_uint), ("ne", ctypes.c_int64 * 4), ("contiguous", ctypes.c_int),
                ("nb", ctypes.c_size_t * 4)]

    @classmethod
    def of(cls, type_, ne, contiguous=True, nb=None):
        """ne (padded with 1s to four dimensions); nb defaults to ggml's contiguous strides"""
        ne = list(ne) + [1] * (4 - len(ne))
        if nb is None:
            size, blck = GGML_TYPE_BLOCK[type_]
            nb = [size, size * (ne[0] // blck)]
            nb += [nb[1] * ne[1], nb[1] * ne[1] * ne[2]]
        nb = list(nb) + [0] * (4 - len(nb))
        return cls(type_, (ctypes.c_int64 * 4)(*ne), int(contiguous), (ctypes.c_size_t * 4)(*nb))

    @classmethod
    def of_tensor(cls, t):
        """ggml view of a torch tensor of up to four dimensions: ne reversed from
        its shape, nb from its strides (in bytes), ggml's order"""
        import torch
        types = {torch.float32: GGML_F32, torch.float16: GGML_F16, torch.int32: GGML_I32}
        es = t.element_size()
        ne = list(reversed(t.shape)) + [1] * (4 - t.dim())
        nb = [st * es for st in reversed(t.stride())]
        for d in range(t.dim(), 4):  # missing outer dimensions: ggml's contiguous extension
            nb.append(nb[-1] * ne[d - 1] if nb else es)
        return cls(types[t.dtype], (ctypes.c_int64 * 4)(*ne), int(t.is_contiguous()), (ctypes.c_size_t * 4)(*nb))


class Exl3Error(RuntimeError):
    def __init__(self, status, what):
        self.status = status
        super().__init__(f"{what}: status {status}")


def load(path=LIB_PATH):
    if not Path(path).exists():
        raise ImportError(f"{path} is not built (run __graft_entry__.build() or make -C xiaomi-hexagon-exl3_amd)")
    L = ctypes.CDLL(str(path))
    vp, sz, u, i, st = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint, ctypes.c_int, ctypes.c_void_p
    L.exl3_hip_version.restype = u
    L.exl3_hip_version.argtypes = []
    L.exl3_hip_status_string.restype = ctypes.c_char_p
    L.exl3_hip_status_string.argtypes = [i]
    L.exl3_hip_gemv_max_rows.restype = sz
    L.exl3_hip_gemv_max_rows.argtypes = []
    L.exl3_hip_supports_mul_mat.restype = i
    L.exl3_hip_supports_mul_mat.argtypes = [u, u, sz, sz, sz, i, i]
    L.exl3_hip_mul_mat_workspace_bytes.restype = sz
    L.exl3_hip_mul_mat_workspace_bytes.argtypes = [sz, sz, sz]
    L.exl3_hip_workspace_init.restype = i
    L.exl3_hip_workspace_init.argtypes = [vp, sz, st]
    L.exl3_hip_mul_mat.restype = i
    L.exl3_hip_mul_mat.argtypes = [vp, u, u, sz, sz, vp, i, sz, sz, vp, i, sz, vp, sz, st]
    L.exl3_hip_mul_mat_noalloc.restype = i
    L.exl3_hip_mul_mat_noalloc.argtypes = [vp, u, u, sz, sz, vp, i, sz, sz, vp, i, sz, st]
    L.exl3_hip_mul_mat_add.restype = i
    L.exl3_hip_decode_batch.restype = i
    L.exl3_hip_decode_batch.argtypes = [vp, sz, i, u, st]
    L.exl3_hip_mul_mat_add.argtypes = [vp, u, u, sz, sz, vp, i, sz, sz, vp, sz, vp, i, sz, vp, sz, st]
    L.exl3_hip_mul_mat_group.restype = i
    L.exl3_hip_mul_mat_group.argtypes = [vp, sz, u, u, sz, vp, i, sz, sz, i, vp, sz, st]
    L.exl3_hip_decode.restype = i
    L.exl3_hip_decode.argtypes = [vp, i, u, u, sz, sz, sz, sz, vp, st]
    L.exl3_hip_reconstruct.restype = i
    L.exl3_hip_reconstruct.argtypes = [vp, i, vp, vp, u, u, sz, sz, sz, sz, vp, st]
    L.exl3_hip_get_rows.restype = i
    L.exl3_hip_get_rows.argtypes = [vp, u, u, sz, sz, vp, sz, vp, i, sz, vp, st]
    L.exl3_hip_model_open.restype = vp
    L.exl3_hip_model_open.argtypes = [ctypes.c_char_p, ctypes.c_char_p, sz]
    L.exl3_hip_model_close.restype = None
    L.exl3_hip_model_close.argtypes = [vp]
    for fn in ("tensor_count", "payload_bytes", "hidden_size", "vocab_size", "matrix_count"):
        getattr(L, "exl3_hip_model_" + fn).restype = sz
        getattr(L, "exl3_hip_model_" + fn).argtypes = [vp]
    L.exl3_hip_model_bits_per_weight.restype = ctypes.c_double
    L.exl3_hip_model_bits_per_weight.argtypes = [vp]
    L.exl3_hip_model_embedding.restype = i
    L.exl3_hip_model_embedding.argtypes = [vp, ctypes.c_uint32, vp]
    L.exl3_hip_model_matrix.restype = i
    L.exl3_hip_model_matrix.argtypes = [vp, sz, ctypes.c_char_p, sz, ctypes.POINTER(u), ctypes.POINTER(u),
                                        ctypes.POINTER(sz), ctypes.POINTER(sz)]
    L.exl3_hip_model_record_bytes.restype = sz
    L.exl3_hip_model_record_bytes.argtypes = [vp, sz]
    L.exl3_hip_model_upload_records.restype = i
    L.exl3_hip_model_upload_records.argtypes = [vp, sz, vp, st]
    L.exl3_hip_codebook.restype = i
    L.exl3_hip_codebook.argtypes = [vp, sz, u, vp, st]
    L.exl3_hip_hadamard128.restype = i
    L.exl3_hip_hadamard128.argtypes = [vp, sz, st]
    L.exl3_hip_pack_records.restype = i
    L.exl3_hip_pack_records.argtypes = [vp, vp, vp, u, sz, sz, vp, st]
    L.exl3_hip_validate_records.restype = i
    L.exl3_hip_validate_records.argtypes = [vp, sz, u, vp, st]
    L.exl3_hip_iface_matmul_workspace_bytes.restype = sz
    L.exl3_hip_iface_matmul_workspace_bytes.argtypes = [u, sz, sz, sz]
    L.exl3_hip_iface_matmul.restype = i
    L.exl3_hip_iface_matmul.argtypes = [u, u, sz, sz, sz, vp, vp, vp, vp, vp, vp, sz, st]
    ti = ctypes.POINTER(TensorInfo)
    L.exl3_hip_supports_op.restype = i
    L.exl3_hip_supports_op.argtypes = [i, ti, ti, ti]
    L.exl3_hip_mul_mat_nd.restype = i
    L.exl3_hip_mul_mat_nd.argtypes = [vp, u, u, sz, sz, vp, ti, vp, ti, vp, sz, st]
    L.exl3_hip_get_rows_nd.restype = i
    L.exl3_hip_get_rows_nd.argtypes = [vp, u, u, sz, sz, vp, ti, vp, ti, vp, st]
    L.exl3_hip_workspace_status.restype = i
    L.exl3_hip_workspace_status.argtypes = [vp, sz, ctypes.POINTER(i), st]
    L.exl3_hip_test_exchange_fault.restype = i
    L.exl3_hip_test_exchange_fault.argtypes = [i, i]
    L.exl3_hip_mul_mat_group_workspace_bytes.restype = sz
    L.exl3_hip_mul_mat_group_workspace_bytes.argtypes = [sz, ctypes.POINTER(sz), sz, sz]
    L.exl3_hip_model_embedding_tables.restype = i
    L.exl3_hip_model_embedding_tables.argtypes = [vp, ctypes.POINTER(sz), ctypes.c_char_p, sz]
    L.exl3_hip_model_embedding_table.restype = i
    L.exl3_hip_model_embedding_table.argtypes = [vp, sz, ctypes.c_char_p, sz, ctypes.POINTER(sz), ctypes.POINTER(sz),
                                                 ctypes.POINTER(u), ctypes.POINTER(sz)]
    return L


_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        _LIB = load()
    return _LIB


def _stream(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _check(status, what):
    if status != OK:
        raise Exl3Error(status, what)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def workspace_bytes(k, n, rows):
    return lib().exl3_hip_mul_mat_workspace_bytes(k, n, rows)


def new_workspace(k, n, rows, device="cuda", nbytes=None):
    """A zero-initialised workspace for calls up to (k, n, rows), or of nbytes
    (for instance group_workspace_bytes of a grouped call) when given."""
    import torch
    nbytes = max(256, workspace_bytes(k, n, rows) if nbytes is None else nbytes)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    _check(lib().exl3_hip_workspace_init(_ptr(ws), nbytes, _stream()), "workspace_init")
    return ws


def workspace_faulted(workspace=None, stream=None):
    """exl3_hip_workspace_status: True when a split-K hand-off with this workspace (None:
    the internal one of this stream) gave up waiting; clear with workspace_init"""
    f = ctypes.c_int()
    wb = workspace.numel() if workspace is not None else 0
    _check(lib().exl3_hip_workspace_status(_ptr(workspace), wb, ctypes.byref(f), _stream(stream)), "workspace_status")
    return bool(f.value)


def workspace_init(workspace=None, stream=None):
    wb = workspace.numel() if workspace is not None else 0
    _check(lib().exl3_hip_workspace_init(_ptr(workspace), wb, _stream(stream)), "workspace_init")


def mul_mat(records, bits, k, n, x, codebook=CB_MUL1, out_dtype=None, y=None, workspace=None, stream=None,
            residual=None):
    """y = EXL3 linear layer applied to x ([rows, k] fp16/fp32 CUDA tensor, row stride x.stride(0)).
    residual ([rows, n], y's dtype; may be y itself): y = residual + layer(x) in one call
    (exl3_hip_mul_mat_add)."""
    import torch
    assert x.dim() == 2 and x.stride(1) == 1 and x.dtype in (torch.float16, torch.float32)
    rows = x.shape[0]
    if y is None:
        dt = out_dtype or (residual.dtype if residual is not None else torch.float32)
        y = torch.empty((rows, n), dtype=dt, device=x.device)
    assert y.dim() == 2 and y.stride(1) == 1 and y.dtype in (torch.float16, torch.float32)
    xt = F16 if x.dtype == torch.float16 else F32
    yt = F16 if y.dtype == torch.float16 else F32
    ws_ptr, ws_bytes = (None, 0) if workspace is None else (_ptr(workspace), workspace.numel())
    if residual is None:
        _check(lib().exl3_hip_mul_mat(_ptr(records), bits, codebook, k, n, _ptr(x), xt, rows, x.stride(0), _ptr(y),
                                      yt, y.stride(0), ws_ptr, ws_bytes, _stream(stream)), "mul_mat")
        return y
    assert residual.dim() == 2 and residual.stride(1) == 1 and residual.dtype == y.dtype
    _check(lib().exl3_hip_mul_mat_add(_ptr(records), bits, codebook, k, n, _ptr(x), xt, rows, x.stride(0),
                                      _ptr(residual), residual.stride(0), _ptr(y), yt, y.stride(0), ws_ptr, ws_bytes,
                                      _stream(stream)), "mul_mat_add")
    return y


class _MatrixDesc(ctypes.Structure):
    _fields_ = [("records", ctypes.c_void_p), ("n", ctypes.c_size_t), ("y", ctypes.c_void_p),
                ("y_row_stride", ctypes.c_size_t)]


def mul_mat_group(mats, bits, k, x, codebook=CB_MUL1, out_dtype=None, workspace=None, stream=None):
    """[y_i] = layer_i(x) for matrices [(records_i, n_i)] (or (records_i, n_i, y_i)) sharing k, bits, codebook
    and x: one GEMV launch at rows <= exl3_hip_gemv_max_rows() (32)."""
    import torch
    assert x.dim() == 2 and x.stride(1) == 1 and x.dtype in (torch.float16, torch.float32)
    rows = x.shape[0]
    ys, descs = [], (_MatrixDesc * len(mats))()
    for idx, m in enumerate(mats):
        rec, n = m[0], m[1]
        y = m[2] if len(m) > 2 else torch.empty((rows, n), dtype=out_dtype or torch.float32, device=x.device)
        assert y.dim() == 2 and y.stride(1) == 1
        descs[idx] = _MatrixDesc(rec.data_ptr(), n, y.data_ptr(), y.stride(0))
        ys.append(y)
    yt = F16 if ys[0].dtype == torch.float16 else F32
    assert all(y.dtype == ys[0].dtype for y in ys)
    xt = F16 if x.dtype == torch.float16 else F32
    ws_ptr, ws_bytes = (None, 0) if workspace is None else (_ptr(workspace), workspace.numel())
    _check(lib().exl3_hip_mul_mat_group(ctypes.cast(descs, ctypes.c_void_p), len(mats), bits, codebook, k, _ptr(x), xt,
                                        rows, x.stride(0), yt, ws_ptr, ws_bytes, _stream(stream)), "mul_mat_group")
    return ys


def decode(src, bits, k, n, codebook=CB_MUL1, layout=LAYOUT_UPSTREAM_TILES, first=0, count=None, out=None,
           stream=None):
    """Row-major fp16 bits (int16 tensor [k, count]) of the decoded trellis weights."""
    import torch
    count = n if count is None else count
    if out is None:
        out = torch.empty((k, count), dtype=torch.int16, device=src.device)
    _check(lib().exl3_hip_decode(_ptr(src), layout, bits, codebook, k, n, first, count, _ptr(out), _stream(stream)),
           "decode")
    return out


class _DecodeDesc(ctypes.Structure):
    _fields_ = [("src", ctypes.c_void_p), ("k", ctypes.c_size_t), ("n", ctypes.c_size_t),
                ("out", ctypes.c_void_p), ("bits", ctypes.c_uint)]


def decode_batch(items, codebook=CB_MUL1, layout=LAYOUT_UPSTREAM_TILES, stream=None):
    """items: [(src, bits, k, n, out)] with out an int16 tensor [k, n] (or None to allocate).
    Decodes every matrix (exl3_hip_decode_batch); returns the outputs."""
    import torch
    outs, descs = [], (_DecodeDesc * max(1, len(items)))()
    for j, (src, bits, k, n, out) in enumerate(items):
        if out is None:
            out = torch.empty((k, n), dtype=torch.int16, device=src.device)
        outs.append(out)
        descs[j] = _DecodeDesc(src.data_ptr(), k, n, out.data_ptr(), bits)
    _check(lib().exl3_hip_decode_batch(ctypes.cast(descs, ctypes.c_void_p), len(items), layout, codebook,
                                       _stream(stream)), "decode_batch")
    return outs


def reconstruct(src, bits, k, n, su=None, sv=None, codebook=CB_MUL1, layout=LAYOUT_UPSTREAM_TILES, first=0,
                count=None, out=None, stream=None):
    import torch
    count = n if count is None else count
    if out is None:
        out = torch.empty((k, count), dtype=torch.int16, device=src.device)
    _check(lib().exl3_hip_reconstruct(_ptr(src), layout, _ptr(su), _ptr(sv), bits, codebook, k, n, first, count,
                                      _ptr(out), _stream(stream)), "reconstruct")
    return out


def get_rows(records, bits, k, n, ids, codebook=CB_MUL1, out_dtype=None, out=None, bad_ids=None, stream=None):
    """GET_ROWS (ggml_exl3_get_rows): out[r] = column ids[r] of the original-basis
    weight, [count, k] fp32 (ggml's dst type) or fp16.  ids: int32 CUDA tensor.
    bad_ids: optional int32 CUDA tensor of one element, set to 1 when an id is
    outside [0, n) (that row is NaN)."""
    import torch
    assert ids.dtype == torch.int32 and ids.is_contiguous()
    count = ids.numel()
    if out is None:
        out = torch.empty((count, k), dtype=out_dtype or torch.float32, device=ids.device)
    assert out.dim() == 2 and out.stride(1) == 1 and out.dtype in (torch.float16, torch.float32)
    ot = F16 if out.dtype == torch.float16 else F32
    _check(lib().exl3_hip_get_rows(_ptr(records), bits, codebook, k, n, _ptr(ids), count, _ptr(out), ot,
                                   out.stride(0), _ptr(bad_ids), _stream(stream)), "get_rows")
    return out


def mul_mat_nd(records, bits, k, n, x, y, codebook=CB_MUL1, workspace=None, stream=None):
    """The ggml op on ggml views (exl3_hip_mul_mat_nd): x is a torch tensor of up to four
    dimensions whose last dimension (ggml's ne[0]) is k and dense, y the same shape with n;
    both may be permuted or sliced views.  Every row of x is multiplied into the row of y
    with the same indices, the rows addressed as the reference's row_offset does."""
    xi, yi = TensorInfo.of_tensor(x), TensorInfo.of_tensor(y)
    ws_ptr, ws_bytes = (None, 0) if workspace is None else (_ptr(workspace), workspace.numel())
    _check(lib().exl3_hip_mul_mat_nd(_ptr(records), bits, codebook, k, n, _ptr(x), ctypes.byref(xi), _ptr(y),
                                     ctypes.byref(yi), ws_ptr, ws_bytes, _stream(stream)), "mul_mat_nd")
    return y


def get_rows_nd(records, bits, k, n, ids, out, codebook=CB_MUL1, bad_ids=None, stream=None):
    """GET_ROWS on ggml views (exl3_hip_get_rows_nd): ids an int32 tensor of up to three
    dimensions (any strides), out of shape ids.shape + (k,) (any disjoint row strides)."""
    ii, oi = TensorInfo.of_tensor(ids), TensorInfo.of_tensor(out)
    _check(lib().exl3_hip_get_rows_nd(_ptr(records), bits, codebook, k, n, _ptr(ids), ctypes.byref(ii), _ptr(out),
                                      ctypes.byref(oi), _ptr(bad_ids), _stream(stream)), "get_rows_nd")
    return out


def group_workspace_bytes(k, ns, rows):
    arr = (ctypes.c_size_t * len(ns))(*ns)
    return lib().exl3_hip_mul_mat_group_workspace_bytes(k, arr, len(ns), rows)


class Model:
    """exl3::Model (src/exl3_model.cpp:79-187) through the C-ABI: the deployment
    reader of a directory with model.safetensors and hexagon-exl3.json.  Raises
    Exl3Error (status INVAL_PARAMS) with the reader's reason when the model is
    malformed."""

    def __init__(self, directory):
        err = ctypes.create_string_buffer(512)
        h = lib().exl3_hip_model_open(str(directory).encode(), err, len(err))
        if not h:
            raise Exl3Error(1, "model_open: " + err.value.decode(errors="replace"))
        self._h = h

    def close(self):
        if self._h:
            lib().exl3_hip_model_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    tensor_count = property(lambda self: lib().exl3_hip_model_tensor_count(self._h))
    payload_bytes = property(lambda self: lib().exl3_hip_model_payload_bytes(self._h))
    hidden_size = property(lambda self: lib().exl3_hip_model_hidden_size(self._h))
    vocab_size = property(lambda self: lib().exl3_hip_model_vocab_size(self._h))
    bits_per_weight = property(lambda self: lib().exl3_hip_model_bits_per_weight(self._h))

    def embedding(self, token):
        """fp16 bits (numpy uint16 [hidden_size]) of token's tied embedding"""
        import numpy as np
        out = np.zeros(self.hidden_size, dtype=np.uint16)
        _check(lib().exl3_hip_model_embedding(self._h, token, out.ctypes.data_as(ctypes.c_void_p)), "model_embedding")
        return out

    def matrices(self):
        """[(prefix, bits, codebook, k, n)] of every EXL3 matrix, in name order"""
        out = []
        for idx in range(lib().exl3_hip_model_matrix_count(self._h)):
            name = ctypes.create_string_buffer(1024)
            b, c = ctypes.c_uint(), ctypes.c_uint()
            kk, nn = ctypes.c_size_t(), ctypes.c_size_t()
            _check(lib().exl3_hip_model_matrix(self._h, idx, name, len(name), ctypes.byref(b), ctypes.byref(c),
                                               ctypes.byref(kk), ctypes.byref(nn)), "model_matrix")
            out.append((name.value.decode(), b.value, c.value, kk.value, nn.value))
        return out

    def embedding_tables(self):
        """[(prefix, rows, groups, bits, width_padded)] of the row-coded embedding
        tables; raises Exl3Error with the audit's reason for a malformed one"""
        count = ctypes.c_size_t()
        err = ctypes.create_string_buffer(512)
        st = lib().exl3_hip_model_embedding_tables(self._h, ctypes.byref(count), err, len(err))
        if st != OK:
            raise Exl3Error(st, "model_embedding_tables: " + err.value.decode(errors="replace"))
        out = []
        for idx in range(count.value):
            name = ctypes.create_string_buffer(1024)
            rows, groups, width = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
            bits = ctypes.c_uint()
            _check(lib().exl3_hip_model_embedding_table(self._h, idx, name, len(name), ctypes.byref(rows),
                                                        ctypes.byref(groups), ctypes.byref(bits), ctypes.byref(width)),
                   "model_embedding_table")
            out.append((name.value.decode(), rows.value, groups.value, bits.value, width.value))
        return out

    def upload_records(self, index, device="cuda", stream=None):
        """uint8 CUDA tensor of matrix index's group records (for mul_mat)"""
        import torch
        nbytes = lib().exl3_hip_model_record_bytes(self._h, index)
        rec = torch.empty(nbytes, dtype=torch.uint8, device=device)
        _check(lib().exl3_hip_model_upload_records(self._h, index, _ptr(rec), _stream(stream)), "model_upload_records")
        return rec


def supports_op(op, dst, src0, src1=None):
    """exl3_hip_supports_op: 1 served, 0 refused, -1 no EXL3 tensor involved"""
    return lib().exl3_hip_supports_op(op, ctypes.byref(dst), ctypes.byref(src0),
                                      ctypes.byref(src1) if src1 is not None else None)


def codebook_values(states, codebook, out=None, stream=None):
    import torch
    if out is None:
        out = torch.empty_like(states)
    _check(lib().exl3_hip_codebook(_ptr(states), states.numel(), codebook, _ptr(out), _stream(stream)), "codebook")
    return out


def hadamard128(values, stream=None):
    _check(lib().exl3_hip_hadamard128(_ptr(values), values.numel(), _stream(stream)), "hadamard128")
    return values


def pack_records(packed, su, sv, bits, k, n, out=None, stream=None):
    import torch
    if out is None:
        out = torch.empty(((n // 128) * (k // 128) * (2048 * bits + 512),), dtype=torch.uint8, device=packed.device)
    _check(lib().exl3_hip_pack_records(_ptr(packed), _ptr(su), _ptr(sv), bits, k, n, _ptr(out), _stream(stream)),
           "pack_records")
    return out


def iface_matmul(packed, suh, svh, x, bits, k, n, codebook=CB_MUL1, y=None, workspace=None, stream=None):
    """The DSP service's layer (exl3_iface_matmul): upstream tiles [k/16, n/16, 16 bits] int16/uint16,
    su [k] and sv [n] fp16, x [batch, k] fp32 (dense) -> y [batch, n] fp32, in one call."""
    import torch
    assert x.dim() == 2 and x.dtype == torch.float32 and x.is_contiguous() and x.shape[1] == k
    if y is None:
        y = torch.empty((x.shape[0], n), dtype=torch.float32, device=x.device)
    assert y.dtype == torch.float32 and y.is_contiguous() and tuple(y.shape) == (x.shape[0], n)
    wb = workspace.numel() if workspace is not None else 0
    _check(lib().exl3_hip_iface_matmul(bits, codebook, k, n, x.shape[0], _ptr(packed), _ptr(suh), _ptr(svh), _ptr(x),
                                       _ptr(y), _ptr(workspace), wb, _stream(stream)), "iface_matmul")
    return y


def new_iface_workspace(bits, k, n, batch, device="cuda"):
    import torch
    nbytes = lib().exl3_hip_iface_matmul_workspace_bytes(bits, k, n, batch)
    if not nbytes:
        raise Exl3Error(INVAL_PARAMS, "iface_matmul_workspace_bytes")
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    _check(lib().exl3_hip_workspace_init(_ptr(ws), nbytes, _stream()), "workspace_init")
    return ws


def validate_records(records, bits, stream=None):
    import torch
    res = torch.empty(1, dtype=torch.int32, device=records.device)
    _check(lib().exl3_hip_validate_records(_ptr(records), records.numel(), bits, _ptr(res), _stream(stream)),
           "validate_records")
    return int(res.item())
