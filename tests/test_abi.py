"""CPU checks of the drop-in boundary: the product library loads and exports
every function include/*.h declares; the oracle agrees with the compiled
reference codec (when the reference build exists)."""
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "xiaomi-hexagon-exl3_amd" / "libexl3_hip.so"


def declared_c_functions():
    text = (ROOT / "include" / "exl3_hip.h").read_text()
    return sorted(set(re.findall(r"\b(exl3_hip_\w+)\s*\(", text)))


def exported_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB)], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


def test_library_loads_and_exports_c_abi():
    import conftest
    amd = conftest.load_amd()   # loads libexl3_hip.so, binds every prototype; no GPU call
    syms = exported_symbols()
    declared = declared_c_functions()
    assert len(declared) >= 13
    missing = [f for f in declared if f not in syms]
    assert not missing, missing
    assert set(amd.EXPORTS) == set(declared)
    assert amd.lib().exl3_hip_version() == 10100
    assert amd.lib().exl3_hip_gemv_max_rows() == 32


def test_library_exports_codec_api():
    out = subprocess.run(["nm", "-DC", "--defined-only", str(LIB)], capture_output=True, text=True, check=True).stdout
    text = (ROOT / "include" / "exl3_codec.h").read_text()
    names = sorted(set(re.findall(r"^\w[\w\s\*]*?\b(\w+)\(", text, re.M)))
    assert {"decode_inner", "reconstruct_slice", "hadamard128", "decode_codebook"} <= set(names)
    for name in names:
        assert f"exl3::{name}(" in out, name


def test_host_side_status_and_planning():
    import conftest
    L = conftest.load_amd().lib()
    # pure host logic, no device work
    assert L.exl3_hip_supports_mul_mat(4, 2, 14336, 4096, 1, 1, 1) == 1
    assert L.exl3_hip_supports_mul_mat(0, 2, 14336, 4096, 1, 1, 1) == 0
    assert L.exl3_hip_supports_mul_mat(4, 3, 14336, 4096, 1, 1, 1) == 0
    assert L.exl3_hip_supports_mul_mat(4, 2, 14300, 4096, 1, 1, 1) == 0
    assert L.exl3_hip_supports_mul_mat(4, 2, 128, 128, 0, 1, 1) == 0
    assert L.exl3_hip_mul_mat_workspace_bytes(14336, 4096, 1) > 0
    assert L.exl3_hip_mul_mat_workspace_bytes(14336, 4096, 512) > L.exl3_hip_mul_mat_workspace_bytes(14336, 4096, 8)
    assert L.exl3_hip_mul_mat_workspace_bytes(100, 4096, 1) == 0
    # rows 17..32: the grouped GEMV's prepared activations (4 matrices x 112 records x 256 B per row)
    # are in it, beyond what GEMV calls of up to 8 rows need
    assert (L.exl3_hip_mul_mat_workspace_bytes(14336, 4096, 32) >=
            L.exl3_hip_mul_mat_workspace_bytes(14336, 4096, 8) + 4 * 112 * 256 * 32)
    # rejected arguments never reach the device
    assert L.exl3_hip_mul_mat(None, 4, 2, 128, 128, None, 1, 1, 128, None, 0, 128, None, 0, None) == 1
    assert L.exl3_hip_decode(None, 0, 4, 2, 16, 16, 0, 16, None, None) == 1
    assert L.exl3_hip_get_rows(None, 4, 2, 128, 128, None, 1, None, 0, 128, None, None) == 1
    assert L.exl3_hip_mul_mat_group(None, 1, 4, 2, 2048, None, 1, 1, 2048, 1, None, 0, None) == 1
    # fused residual add: NULL residual, short residual stride, misaligned residual
    assert L.exl3_hip_mul_mat_add(None, 4, 2, 128, 128, None, 1, 1, 128, None, 128, 0x100000, 0, 128, None, 0,
                                  None) == 1
    assert L.exl3_hip_mul_mat_add(None, 4, 2, 128, 128, None, 1, 1, 128, 0x200000, 64, 0x100000, 0, 128, None, 0,
                                  None) == 1
    assert L.exl3_hip_mul_mat_add(None, 4, 2, 128, 128, None, 1, 1, 128, 0x200002, 128, 0x100000, 0, 128, None, 0,
                                  None) == 1
    import ctypes
    descs = (ctypes.c_size_t * 4)(0, 128, 0, 128)   # one descriptor: NULL records
    assert L.exl3_hip_mul_mat_group(ctypes.cast(descs, ctypes.c_void_p), 0, 4, 2, 128, None, 1, 1, 128, 1,
                                    None, 0, None) == 1   # count 0
    assert L.exl3_hip_mul_mat_group(ctypes.cast(descs, ctypes.c_void_p), 5, 4, 2, 128, None, 1, 1, 128, 1,
                                    None, 0, None) == 1   # more than 4 matrices
    assert L.exl3_hip_mul_mat_group(ctypes.cast(descs, ctypes.c_void_p), 1, 4, 2, 128, None, 1, 1, 128, 1,
                                    None, 0, None) == 1   # NULL records
    assert L.exl3_hip_get_rows(None, 4, 2, 100, 128, None, 1, None, 0, 128, None, None) == 1
    assert L.exl3_hip_get_rows(None, 4, 2, 128, 128, None, 0, None, 0, 128, None, None) == 0  # count 0: no-op
    assert L.exl3_hip_hadamard128(None, 100, None) == 1
    assert L.exl3_hip_decode_batch(None, 0, 0, 2, None) == 0        # nothing to decode
    assert L.exl3_hip_decode_batch(None, 1, 0, 2, None) == 1        # NULL descriptors
    assert L.exl3_hip_decode_batch(None, 0, 7, 2, None) == 1        # unknown layout
    bad = (ctypes.c_size_t * 5)(0x10000, 16, 16, 0x20000, 9)        # bits 9
    assert L.exl3_hip_decode_batch(ctypes.cast(bad, ctypes.c_void_p), 1, 0, 2, None) == 1
    bad = (ctypes.c_size_t * 5)(0x10000, 16, 24, 0x20000, 4)        # n not a multiple of 16
    assert L.exl3_hip_decode_batch(ctypes.cast(bad, ctypes.c_void_p), 1, 0, 2, None) == 1
    assert L.exl3_hip_status_string(3) == b"workspace too small"
    # the DSP service's layer on upstream tiles: its argument checks, then workspace sizing
    assert L.exl3_hip_iface_matmul(4, 2, 128, 128, 1, None, None, None, None, None, None, 0, None) == 1  # NULLs
    for bits, cb, k, n, batch in ((0, 2, 128, 128, 1), (9, 2, 128, 128, 1), (4, 3, 128, 128, 1),
                                  (4, 2, 100, 128, 1), (4, 2, 128, 96, 1), (4, 2, 128, 128, 0)):
        assert L.exl3_hip_iface_matmul(bits, cb, k, n, batch, 0x10000, 0x20000, 0x30000, 0x40000, 0x50000,
                                       None, 0, None) == 1, (bits, cb, k, n, batch)
        if cb <= 2:  # the workspace size does not depend on the codebook
            assert L.exl3_hip_iface_matmul_workspace_bytes(bits, k, n, batch) == 0
    assert L.exl3_hip_iface_matmul(4, 2, 128, 128, 1, 0x10008, 0x20000, 0x30000, 0x40000, 0x50000,
                                   None, 0, None) == 1   # packed not 16-byte aligned
    ws = L.exl3_hip_iface_matmul_workspace_bytes(4, 14336, 4096, 8)
    assert ws >= L.exl3_hip_mul_mat_workspace_bytes(14336, 4096, 8) + 3584 * (2048 * 4 + 512)
    assert L.exl3_hip_iface_matmul(4, 2, 14336, 4096, 8, 0x10000, 0x20000, 0x30000, 0x40000, 0x50000,
                                   0x100000, ws - 1, None) == 3   # caller workspace too small


@pytest.mark.skipif(not (ROOT / "oracle" / "_ref" / "check_ref").exists(), reason="reference build absent")
def test_oracle_exhaustive_vs_compiled_reference():
    r = subprocess.run([str(ROOT / "oracle" / "_ref" / "check_ref")], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 mismatches over 2^32" in r.stdout


def test_ggml_op_predicates():
    """exl3_hip_supports_op: the supports_op rules the reference applies to ops that
    touch an EXL3 tensor (patches/llama-exl3.patch:69-97), one accepted and one
    refused case per rule, and -1 for ops without an EXL3 tensor."""
    import conftest
    a = conftest.load_amd()
    T = a.TensorInfo.of
    F32, F16, I32, Q4, Q6, Q8 = a.GGML_F32, a.GGML_F16, a.GGML_I32, 43, 44, 45
    k, n, rows = 2048, 6144, 7
    w = T(Q4, [k, n])
    # MUL_MAT (patch:81-84): 128-multiple 2-D contiguous weight, F32/F16 activations
    assert a.supports_op(a.OP_MUL_MAT, T(F32, [n, rows]), w, T(F32, [k, rows])) == 1
    assert a.supports_op(a.OP_MUL_MAT, T(F32, [n, rows]), T(Q8, [k, n]), T(F16, [k, rows])) == 1
    assert a.supports_op(a.OP_MUL_MAT, T(F32, [n, 2, 3]), T(Q6, [k, n]), T(F16, [k, 2, 3])) == 1   # batched rows
    assert a.supports_op(a.OP_MUL_MAT, T(F32, [n, rows]), w, T(30, [k, rows])) == 0               # BF16 input
    assert a.supports_op(a.OP_MUL_MAT, T(F32, [n, rows]), T(Q4, [k + 64, n]), T(F32, [k + 64, rows])) == 0
    assert a.supports_op(a.OP_MUL_MAT, T(F32, [n, rows]), T(Q4, [k, n - 16]), T(F32, [k, rows])) == 0
    assert a.supports_op(a.OP_MUL_MAT, T(F32, [n, rows]), T(Q4, [k, n, 2]), T(F32, [k, rows])) == 0  # 3-D weight
    assert a.supports_op(a.OP_MUL_MAT, T(F32, [n, rows]), T(Q4, [k, n], False), T(F32, [k, rows])) == 0
    assert a.supports_op(a.OP_MUL_MAT, T(F16, [n, rows]), w, T(F32, [k, rows])) == 0              # dst not F32
    assert a.supports_op(a.OP_MUL_MAT, T(F32, [n, rows]), w, None) == 0
    assert a.supports_op(a.OP_MUL_MAT, T(F32, [n, rows]), T(F16, [k, n]), T(F32, [k, rows])) == -1
    # MUL_MAT_ID (patch:92-93): never on EXL3 weights
    assert a.supports_op(a.OP_MUL_MAT_ID, T(F32, [n, rows]), w, T(F32, [k, rows])) == 0
    assert a.supports_op(a.OP_MUL_MAT_ID, T(F32, [n, rows]), T(F16, [k, n]), T(F32, [k, rows])) == -1
    # GET_ROWS (patch:94-97): I32 ids into a 128-multiple 2-D table
    assert a.supports_op(a.OP_GET_ROWS, T(F32, [k, 5]), w, T(I32, [5])) == 1
    assert a.supports_op(a.OP_GET_ROWS, T(F16, [k, 5]), w, T(I32, [5])) == 1
    assert a.supports_op(a.OP_GET_ROWS, T(F32, [k, 5]), w, T(27, [5])) == 0                       # I64 ids
    assert a.supports_op(a.OP_GET_ROWS, T(F32, [k, 5]), T(Q4, [k, n, 1, 2]), T(I32, [5])) == 0
    assert a.supports_op(a.OP_GET_ROWS, T(F32, [k, 5]), T(F16, [k, n]), T(I32, [5])) == -1
    # CPY / SET_ROWS (patch:69-72): only a contiguous copy between tensors of one EXL3 type
    assert a.supports_op(a.OP_CPY, T(Q4, [k, n]), w) == 1
    assert a.supports_op(a.OP_CPY, T(Q6, [k, n]), w) == 0                  # type change
    assert a.supports_op(a.OP_CPY, T(F16, [k, n]), w) == 0                 # dequantising copy
    assert a.supports_op(a.OP_CPY, T(Q4, [k, n]), T(F32, [k, n])) == 0     # quantising copy
    assert a.supports_op(a.OP_CPY, T(Q4, [k, n], False), w) == 0
    assert a.supports_op(a.OP_SET_ROWS, T(Q4, [k, n]), T(F32, [k, 3]), T(I32, [3])) == 0
    assert a.supports_op(a.OP_CPY, T(F16, [k, n]), T(F32, [k, n])) == -1


def test_ggml_op_predicates_views():
    """MUL_MAT and GET_ROWS on ggml views: served when every row is addressable as
    the reference's row_offset addresses it (src/exl3-ggml.cpp:11-17, 34-36) by
    exl3_hip_mul_mat_nd / exl3_hip_get_rows_nd; refused when a row cannot be (an
    element stride inside the row, a stride that is not a whole element), when two
    output rows share bytes, or when dst's shape does not follow src0 and src1."""
    import conftest
    a = conftest.load_amd()
    T = a.TensorInfo.of
    F32, F16, I32, Q4 = a.GGML_F32, a.GGML_F16, a.GGML_I32, 43
    k, n = 2048, 6144
    w = T(Q4, [k, n])
    # permuted and sliced 3-D activations: served (one call per non-uniform slice)
    perm = T(F16, [k, 2, 3], nb=[2, 2 * k * 3, 2 * k, 2 * k * 6])
    assert a.supports_op(a.OP_MUL_MAT, T(F32, [n, 2, 3]), w, perm) == 1
    sliced = T(F32, [k, 3, 2], nb=[4, 4 * k, 4 * k * 5, 4 * k * 10])
    assert a.supports_op(a.OP_MUL_MAT, T(F32, [n, 3, 2]), w, sliced) == 1
    # a permuted dst whose rows do not overlap: served
    assert a.supports_op(a.OP_MUL_MAT, T(F32, [n, 2, 3], nb=[4, 4 * n * 3, 4 * n, 4 * n * 6]), w, perm) == 1
    # refused: element stride inside a row, a stride of half an element, overlapping dst rows,
    # dst shape not [ne01, ne11, ne12, ne13]
    assert a.supports_op(a.OP_MUL_MAT, T(F32, [n, 4]), w, T(F32, [k, 4], nb=[8, 8 * k, 32 * k, 32 * k])) == 0
    assert a.supports_op(a.OP_MUL_MAT, T(F32, [n, 4]), w, T(F16, [k, 4], nb=[2, 2 * k + 1, 8 * k + 4, 0])) == 0
    assert a.supports_op(a.OP_MUL_MAT, T(F32, [n, 4], nb=[4, 2 * n, 8 * n, 8 * n]), w, T(F32, [k, 4])) == 0
    assert a.supports_op(a.OP_MUL_MAT, T(F32, [n, 2, 2], nb=[4, 4 * n, 6 * n, 12 * n]), w,
                         T(F32, [k, 2, 2])) == 0   # rows 1 and 2 overlap (stride 1.5 rows)
    assert a.supports_op(a.OP_MUL_MAT, T(F32, [n, 4], nb=[8, 8 * n, 0, 0]), w, T(F32, [k, 4])) == 0
    assert a.supports_op(a.OP_MUL_MAT, T(F32, [n, 5]), w, T(F32, [k, 4])) == 0
    assert a.supports_op(a.OP_MUL_MAT, T(F32, [n + 128, 4]), w, T(F32, [k, 4])) == 0
    assert a.supports_op(a.OP_MUL_MAT, T(F32, [n, 4, 2]), w, T(F32, [k, 8])) == 0
    # GET_ROWS: 2-D ids with strides, their rows into a 3-D dst
    ids2 = T(I32, [3, 2], nb=[8, 24, 48, 48])
    assert a.supports_op(a.OP_GET_ROWS, T(F32, [k, 3, 2]), w, ids2) == 1
    assert a.supports_op(a.OP_GET_ROWS, T(F16, [k, 3, 2], nb=[2, 2 * k + 256, 6 * k + 768, 0]), w, ids2) == 1
    assert a.supports_op(a.OP_GET_ROWS, T(F32, [k, 6]), w, ids2) == 0                    # dst shape
    assert a.supports_op(a.OP_GET_ROWS, T(F32, [k, 3, 2]), w, T(I32, [3, 2], nb=[2, 6, 12, 12])) == 0
    assert a.supports_op(a.OP_GET_ROWS, T(F32, [k, 3, 2], nb=[4, 2 * k, 12 * k, 24 * k]), w, ids2) == 0
    assert a.supports_op(a.OP_GET_ROWS, T(F32, [k, 3, 2]), T(Q4, [k, n], False), ids2) == 0   # strided records


def test_nd_entries_and_group_sizing_host_checks():
    """exl3_hip_mul_mat_nd / _get_rows_nd refuse what their predicates refuse before any
    device work; the group workspace covers the per-matrix GEMM calls of a group."""
    import ctypes
    import conftest
    a = conftest.load_amd()
    L, T = a.lib(), a.TensorInfo.of
    k, n = 2048, 6144
    x, y = T(a.GGML_F32, [k, 4]), T(a.GGML_F32, [n, 4])
    R, X, Y = 0x100000, 0x200000, 0x300000
    assert L.exl3_hip_mul_mat_nd(R, 4, 2, k, n, X, ctypes.byref(T(a.GGML_I32, [k, 4])), Y, ctypes.byref(y),
                                 None, 0, None) == 1
    assert L.exl3_hip_mul_mat_nd(R, 4, 2, k, n, X, ctypes.byref(x), Y,
                                 ctypes.byref(T(a.GGML_F32, [n, 4], nb=[4, 4, 16, 16])), None, 0, None) == 1
    assert L.exl3_hip_mul_mat_nd(R, 4, 2, k, n, X, ctypes.byref(x), Y, ctypes.byref(T(a.GGML_F32, [n, 2, 2])),
                                 None, 0, None) == 1
    assert L.exl3_hip_mul_mat_nd(R, 4, 2, k, n, X, ctypes.byref(x), Y, ctypes.byref(y), 0x400000,
                                 L.exl3_hip_mul_mat_workspace_bytes(k, n, 4) - 1, None) == 3
    assert L.exl3_hip_mul_mat_nd(R, 4, 2, k, n, X, None, Y, ctypes.byref(y), None, 0, None) == 1
    ids = T(a.GGML_I32, [5])
    assert L.exl3_hip_get_rows_nd(R, 4, 2, k, n, X, ctypes.byref(ids), Y,
                                  ctypes.byref(T(a.GGML_F32, [k, 4])), None, None) == 1
    assert L.exl3_hip_get_rows_nd(R, 4, 2, k, n, X, ctypes.byref(T(a.GGML_I32, [0])), Y,
                                  ctypes.byref(T(a.GGML_F32, [k, 0])), None, None) == 0   # no ids: no-op
    # group sizing: gate/up k = 2048, n = 8192 each, at 513 and 520 rows; the GEMM path runs one
    # exl3_hip_mul_mat per matrix, whose split partials may exceed the total width's
    for rows in (513, 520, 33, 8):
        g = a.group_workspace_bytes(2048, [8192, 8192], rows)
        assert g >= L.exl3_hip_mul_mat_workspace_bytes(2048, 8192, rows), rows
        assert g >= L.exl3_hip_mul_mat_workspace_bytes(2048, 16384, rows), rows
    g = a.group_workspace_bytes(4096, [128, 4608], 33)
    assert g >= L.exl3_hip_mul_mat_workspace_bytes(4096, 128, 33)
    assert a.group_workspace_bytes(4096, [128, 4608, 128, 128, 128], 1) == 0   # more than 4 matrices
