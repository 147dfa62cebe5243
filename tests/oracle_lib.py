"""ctypes access to the CPU oracle (oracle/liboracle.so) and, where it was
built, the compiled reference codec (oracle/_ref/libexl3ref.so).
Test infrastructure only."""
import ctypes
import os
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
ORACLE_SO = ROOT / "oracle" / "liboracle.so"
REF_SO = ROOT / "oracle" / "_ref" / "libexl3ref.so"

_u16p = ctypes.POINTER(ctypes.c_uint16)
_f32p = ctypes.POINTER(ctypes.c_float)
_sz = ctypes.c_size_t


def _ptr(a, t=ctypes.c_void_p):
    return ctypes.cast(a.ctypes.data, t)


class Oracle:
    def __init__(self, path=ORACLE_SO):
        if not Path(path).exists():
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = ctypes.CDLL(str(path))
        L.orc_half_to_float.restype = ctypes.c_float
        L.orc_half_to_float.argtypes = [ctypes.c_uint16]
        L.orc_float_to_half.restype = ctypes.c_uint16
        L.orc_float_to_half.argtypes = [ctypes.c_float]
        L.orc_decode_codebook.restype = ctypes.c_uint16
        L.orc_decode_codebook.argtypes = [ctypes.c_uint16, ctypes.c_uint]
        L.orc_decode_tile.argtypes = [_u16p, ctypes.c_uint, ctypes.c_uint, _u16p]
        L.orc_decode_inner_slice.argtypes = [_u16p, _sz, _sz, _sz, _sz, ctypes.c_uint, ctypes.c_uint, _u16p]
        L.orc_decode_inner.argtypes = [_u16p, _sz, _sz, ctypes.c_uint, ctypes.c_uint, _u16p]
        L.orc_hadamard128.argtypes = [_f32p, _sz]
        L.orc_reconstruct_slice.argtypes = [_u16p, _u16p, _u16p, _sz, _sz, _sz, _sz, ctypes.c_uint, ctypes.c_uint, _u16p]
        L.orc_reconstruct.argtypes = [_u16p, _u16p, _u16p, _sz, _sz, ctypes.c_uint, ctypes.c_uint, _u16p]
        L.orc_group_bytes.restype = _sz
        L.orc_group_bytes.argtypes = [ctypes.c_uint]
        L.orc_pack_records.argtypes = [_u16p, _u16p, _u16p, _sz, _sz, ctypes.c_uint, ctypes.c_void_p]
        L.orc_decode_records.argtypes = [ctypes.c_void_p, _sz, _sz, ctypes.c_uint, ctypes.c_uint, _u16p]
        L.orc_validate_records.argtypes = [ctypes.c_void_p, _sz, ctypes.c_uint]
        L.orc_mul_mat.argtypes = [ctypes.c_void_p, ctypes.c_uint, ctypes.c_uint, _sz, _sz, ctypes.c_void_p,
                                  ctypes.c_int, _sz, _sz, _f32p, _sz, ctypes.c_uint]
        L.orc_mul_mat_groups.argtypes = [ctypes.c_void_p, ctypes.c_uint, ctypes.c_uint, _sz, _sz, ctypes.c_void_p,
                                         ctypes.c_int, _sz, _sz, _f32p, _sz, ctypes.c_uint, _sz, _sz]
        L.orc_get_rows.argtypes = [ctypes.c_void_p, ctypes.c_uint, ctypes.c_uint, _sz, _sz, ctypes.c_void_p, _sz,
                                   _f32p, _sz]
        L.orc_iface_matmul.argtypes = [ctypes.c_uint, ctypes.c_uint, _sz, _sz, _sz, _u16p, _u16p, _u16p, _f32p,
                                       _f32p]
        self.L = L

    def codebook_table(self, cb):
        return np.array([self.L.orc_decode_codebook(s, cb) for s in range(65536)], dtype=np.uint16)

    def get_rows(self, records, bits, cb, k, n, ids):
        """ggml_exl3_get_rows: [len(ids), k] float32"""
        r = np.ascontiguousarray(records)
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.zeros((ids.size, k), dtype=np.float32)
        if self.L.orc_get_rows(_ptr(r), bits, cb, k, n, _ptr(ids), ids.size, _ptr(out, _f32p), k):
            raise ValueError("get_rows rejected its arguments")
        return out

    def decode_tile(self, packed, bits, cb):
        p = np.ascontiguousarray(packed, dtype=np.uint16)
        out = np.zeros(256, dtype=np.uint16)
        rc = self.L.orc_decode_tile(_ptr(p, _u16p), bits, cb, _ptr(out, _u16p))
        if rc:
            raise ValueError("decode_tile rejected its arguments")
        return out.reshape(16, 16)

    def decode_inner(self, packed, k, n, bits, cb, first=0, count=None):
        count = n if count is None else count
        p = np.ascontiguousarray(packed, dtype=np.uint16)
        out = np.zeros(k * count, dtype=np.uint16)
        rc = self.L.orc_decode_inner_slice(_ptr(p, _u16p), k, n, first, count, bits, cb, _ptr(out, _u16p))
        if rc:
            raise ValueError("decode_inner rejected its arguments")
        return out.reshape(k, count)

    def hadamard128(self, v):
        a = np.array(v, dtype=np.float32)
        if self.L.orc_hadamard128(_ptr(a, _f32p), a.size):
            raise ValueError("H128 length must be a multiple of 128")
        return a

    def reconstruct(self, packed, su, sv, k, n, bits, cb, first=0, count=None):
        count = n if count is None else count
        p = np.ascontiguousarray(packed, dtype=np.uint16)
        su = np.ascontiguousarray(su).view(np.uint16)
        sv = np.ascontiguousarray(sv).view(np.uint16)
        out = np.zeros(k * count, dtype=np.uint16)
        rc = self.L.orc_reconstruct_slice(_ptr(p, _u16p), _ptr(su, _u16p), _ptr(sv, _u16p), k, n, first, count,
                                          bits, cb, _ptr(out, _u16p))
        if rc:
            raise ValueError("reconstruct rejected its arguments")
        return out.reshape(k, count)

    def pack_records(self, packed, su, sv, k, n, bits):
        p = np.ascontiguousarray(packed, dtype=np.uint16)
        su = np.ascontiguousarray(su).view(np.uint16)
        sv = np.ascontiguousarray(sv).view(np.uint16)
        out = np.zeros((n // 128) * (k // 128) * self.L.orc_group_bytes(bits), dtype=np.uint8)
        if self.L.orc_pack_records(_ptr(p, _u16p), _ptr(su, _u16p), _ptr(sv, _u16p), k, n, bits, _ptr(out)):
            raise ValueError("pack_records rejected its arguments")
        return out

    def decode_records(self, records, k, n, bits, cb):
        r = np.ascontiguousarray(records)
        out = np.zeros(k * n, dtype=np.uint16)
        if self.L.orc_decode_records(_ptr(r), k, n, bits, cb, _ptr(out, _u16p)):
            raise ValueError("decode_records rejected its arguments")
        return out.reshape(k, n)

    def validate_records(self, records, bits):
        r = np.ascontiguousarray(records)
        return self.L.orc_validate_records(_ptr(r), r.nbytes, bits)

    def mul_mat(self, records, bits, cb, k, n, x, threads=1, groups=None):
        """x: [rows, k] float16 or float32 -> y [rows, n] float32"""
        r = np.ascontiguousarray(records)
        x = np.ascontiguousarray(x)
        assert x.dtype in (np.float16, np.float32) and x.shape[1] == k
        rows = x.shape[0]
        y = np.zeros((rows, n), dtype=np.float32)
        if groups is None:
            rc = self.L.orc_mul_mat(_ptr(r), bits, cb, k, n, _ptr(x), int(x.dtype == np.float16), rows,
                                    x.strides[0], _ptr(y, _f32p), y.strides[0], threads)
        else:
            rc = self.L.orc_mul_mat_groups(_ptr(r), bits, cb, k, n, _ptr(x), int(x.dtype == np.float16), rows,
                                           x.strides[0], _ptr(y, _f32p), y.strides[0], threads, groups[0], groups[1])
        if rc:
            raise ValueError("mul_mat rejected its arguments")
        return y

    def iface_matmul(self, packed, su, sv, bits, cb, k, n, x):
        """The DSP service's layer: upstream tiles + separate su/sv, x [batch, k] fp32 -> y [batch, n] fp32"""
        p = np.ascontiguousarray(packed, dtype=np.uint16)
        su = np.ascontiguousarray(su).view(np.uint16)
        sv = np.ascontiguousarray(sv).view(np.uint16)
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.zeros((x.shape[0], n), dtype=np.float32)
        if self.L.orc_iface_matmul(bits, cb, k, n, x.shape[0], _ptr(p, _u16p), _ptr(su, _u16p), _ptr(sv, _u16p),
                                   _ptr(x, _f32p), _ptr(y, _f32p)):
            raise ValueError("iface_matmul rejected its arguments")
        return y



class Reference:
    """The reference codec compiled from its own sources (oracle/Makefile `ref`)."""

    def __init__(self, path=REF_SO):
        if not Path(path).exists():
            raise FileNotFoundError(f"{path} missing: run `make -C oracle ref`")
        L = ctypes.CDLL(str(path))
        L.ref_half_to_float.restype = ctypes.c_float
        L.ref_half_to_float.argtypes = [ctypes.c_uint16]
        L.ref_float_to_half.restype = ctypes.c_uint16
        L.ref_float_to_half.argtypes = [ctypes.c_float]
        L.ref_decode_codebook.argtypes = [ctypes.c_uint16, ctypes.c_uint, _u16p]
        L.ref_decode_tile.argtypes = [_u16p, ctypes.c_uint, ctypes.c_uint, _u16p]
        L.ref_decode_inner_slice.argtypes = [_u16p, _sz, _sz, _sz, _sz, ctypes.c_uint, ctypes.c_uint, _u16p]
        L.ref_hadamard128.argtypes = [_f32p, _sz]
        L.ref_reconstruct_slice.argtypes = [_u16p, _u16p, _u16p, _sz, _sz, _sz, _sz, ctypes.c_uint, ctypes.c_uint, _u16p]
        self.L = L

    def codebook_table(self, cb):
        out = np.zeros(65536, dtype=np.uint16)
        v = ctypes.c_uint16()
        for s in range(65536):
            if self.L.ref_decode_codebook(s, cb, ctypes.byref(v)):
                raise ValueError("bad codebook")
            out[s] = v.value
        return out

    def decode_tile(self, packed, bits, cb):
        p = np.ascontiguousarray(packed, dtype=np.uint16)
        out = np.zeros(256, dtype=np.uint16)
        if self.L.ref_decode_tile(_ptr(p, _u16p), bits, cb, _ptr(out, _u16p)):
            raise ValueError("rejected")
        return out.reshape(16, 16)

    def decode_inner(self, packed, k, n, bits, cb, first=0, count=None):
        count = n if count is None else count
        p = np.ascontiguousarray(packed, dtype=np.uint16)
        out = np.zeros(k * count, dtype=np.uint16)
        if self.L.ref_decode_inner_slice(_ptr(p, _u16p), k, n, first, count, bits, cb, _ptr(out, _u16p)):
            raise ValueError("rejected")
        return out.reshape(k, count)

    def hadamard128(self, v):
        a = np.array(v, dtype=np.float32)
        if self.L.ref_hadamard128(_ptr(a, _f32p), a.size):
            raise ValueError("rejected")
        return a

    def reconstruct(self, packed, su, sv, k, n, bits, cb, first=0, count=None):
        count = n if count is None else count
        p = np.ascontiguousarray(packed, dtype=np.uint16)
        su = np.ascontiguousarray(su).view(np.uint16)
        sv = np.ascontiguousarray(sv).view(np.uint16)
        out = np.zeros(k * count, dtype=np.uint16)
        if self.L.ref_reconstruct_slice(_ptr(p, _u16p), _ptr(su, _u16p), _ptr(sv, _u16p), k, n, first, count,
                                        bits, cb, _ptr(out, _u16p)):
            raise ValueError("rejected")
        return out.reshape(k, count)
