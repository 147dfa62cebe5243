"""CPU tests that pin the oracle (oracle/exl3_oracle.c) before it is trusted as
the checker: the reference's own known answers, golden vectors made by the
compiled reference codec, closed forms, and planted mistakes."""
import hashlib
import json
import struct
from pathlib import Path

import numpy as np
import pytest

import synth

GOLD = Path(__file__).resolve().parent / "golden"


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def h128_matrix():
    h = np.ones((1, 1))
    while h.shape[0] < 128:
        h = np.block([[h, h], [h, -h]])
    return h / np.sqrt(128.0)


# ---- tests/test_codec.cpp known answers, restated against the oracle -------------

def test_mul1_closed_form_all_states(oracle):
    # tests/test_codec.cpp:16-31: w = rn16((1774 s - 905216) / 2^18), s = byte sum of state * 0x83dcd12d
    st = np.arange(65536, dtype=np.uint64)
    p = (st * np.uint64(0x83DCD12D)) & np.uint64(0xFFFFFFFF)
    s = sum(((p >> np.uint64(8 * b)) & np.uint64(0xFF)).astype(np.int64) for b in range(4))
    exact = (1774 * s - 905216) / 262144.0
    assert np.all(np.abs(exact) >= 2.0 ** -14) and np.all(np.abs(exact) < 65504)
    expect = exact.astype(np.float32).astype(np.float16).view(np.uint16)  # exact in fp32, one RNE to fp16
    got = oracle.codebook_table(2)
    assert np.array_equal(got, expect)


def test_fp16_roundtrip_and_ties(oracle):
    L = oracle.L
    for b in list(range(0, 65536, 7)) + [0x0001, 0x03FF, 0x0400, 0x7BFF, 0x8001, 0xFBFF]:
        if (b & 0x7C00) != 0x7C00:
            assert L.orc_float_to_half(L.orc_half_to_float(b)) == b
    assert L.orc_float_to_half(1.00048828125) == 0x3C00   # tests/test_codec.cpp:63
    assert L.orc_float_to_half(1.00146484375) == 0x3C02   # :64
    assert L.orc_float_to_half(65520.0) == 0x7C00          # :65
    assert L.orc_float_to_half(float("nan")) == 0x7E00
    assert L.orc_float_to_half(-0.0) == 0x8000
    # all halves against numpy's IEEE conversion
    h = np.arange(65536, dtype=np.uint16)
    f = np.array([L.orc_half_to_float(int(v)) for v in h[::97]], dtype=np.float32)
    ref = h[::97].view(np.float16).astype(np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(f[fin].view(np.uint32), ref[fin].view(np.uint32))


def test_float_to_half_matches_numpy_rne(oracle):
    rng = np.random.default_rng(5)
    bits = rng.integers(0, 2 ** 32, 20000, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    fin = np.isfinite(f)
    got = np.array([oracle.L.orc_float_to_half(float(v)) for v in f[fin]], dtype=np.uint16)
    with np.errstate(over="ignore"):
        exp = f[fin].astype(np.float16).view(np.uint16)
    assert np.array_equal(got, exp)


def test_hadamard_involution_and_closed_form(oracle):
    v = np.array([(i % 19 - 9) / 17 for i in range(256)], dtype=np.float32)  # tests/test_codec.cpp:66-71
    twice = oracle.hadamard128(oracle.hadamard128(v))
    assert np.max(np.abs(twice - v)) < 1e-6
    x = synth.normal(3, 384).astype(np.float32)
    H = h128_matrix()
    expect = (x.astype(np.float64).reshape(3, 128) @ H.T).reshape(-1)
    assert np.max(np.abs(oracle.hadamard128(x) - expect)) < 1e-5
    with pytest.raises(ValueError):
        oracle.hadamard128(np.zeros(100, np.float32))


def test_zero_ring_and_rejects(oracle):
    z = np.zeros(128, np.uint16)
    for bits in range(1, 9):
        for cb in range(3):
            t = oracle.decode_tile(z[: 16 * bits], bits, cb)
            assert np.all(t == oracle.L.orc_decode_codebook(0, cb))  # tests/test_codec.cpp:72-80
    with pytest.raises(ValueError):
        oracle.decode_tile(z, 0, 2)                                 # :81-84
    with pytest.raises(ValueError):
        oracle.decode_inner(z, 16, 16, 4, 2, first=16, count=16)    # :85-88


# ---- golden vectors from the compiled reference codec ----------------------------

def test_codebook_golden(oracle):
    g = json.loads((GOLD / "codebook.json").read_text())
    for cb in range(3):
        t = oracle.codebook_table(cb)
        assert sha(t.astype("<u2")) == g[str(cb)]["sha256"]
        assert [int(t[s]) for s in g[str(cb)]["states"]] == g[str(cb)]["values"]


def test_tiles_golden(oracle):
    d = np.load(GOLD / "tiles.npz", allow_pickle=False)
    for bits in range(1, 9):
        for cb in range(3):
            for t in range(d["packed"].shape[2]):
                got = oracle.decode_tile(d["packed"][bits - 1, cb, t, : 16 * bits], bits, cb)
                assert np.array_equal(got.reshape(-1), d["decoded"][bits - 1, cb, t]), (bits, cb, t)


def golden_matrix_inputs(m):
    k, n, bits, seed = m["k"], m["n"], m["bits"], m["seed"]
    p = synth.packed_tiles(seed, k, n, bits)
    su = (synth.uniform01(seed ^ 0x11, k) * 2 - 1).astype(np.float16)
    sv = (synth.uniform01(seed ^ 0x22, n) * 2 - 1).astype(np.float16)
    assert sha(p.astype("<u2")) == m["packed_sha256"] and sha(su) == m["su_sha256"] and sha(sv) == m["sv_sha256"]
    return p, su, sv


@pytest.mark.parametrize("bits", range(1, 9))
def test_matrices_golden(oracle, bits):
    mats = [m for m in json.loads((GOLD / "matrices.json").read_text()) if m["bits"] == bits]
    for m in mats:
        p, su, sv = golden_matrix_inputs(m)
        k, n, cb = m["k"], m["n"], m["cb"]
        inner = oracle.decode_inner(p, k, n, bits, cb)
        assert sha(inner.astype("<u2")) == m["inner_sha256"]
        orig = oracle.reconstruct(p, su, sv, k, n, bits, cb)
        assert sha(orig.astype("<u2")) == m["original_sha256"]
        # slices agree with the full matrix (tools/exl3_verify.cpp:57-66)
        assert np.array_equal(oracle.decode_inner(p, k, n, bits, cb, first=32, count=48), inner[:, 32:80])
        assert np.array_equal(oracle.reconstruct(p, su, sv, k, n, bits, cb, first=128, count=128), orig[:, 128:256])


def test_hadamard_golden(oracle):
    for case in json.loads((GOLD / "hadamard.json").read_text()):
        x = np.array(case["input"], dtype=np.uint32).view(np.float32)
        assert np.array_equal(oracle.hadamard128(x).view(np.uint32), np.array(case["output"], dtype=np.uint32))


def read_exl3ref(path):
    raw = Path(path).read_bytes()
    assert raw[:8] == b"EXL3REF1"
    k, n, bits, cb = struct.unpack("<4I", raw[8:24])
    off = 24
    def take(count):
        nonlocal off
        a = np.frombuffer(raw, dtype="<u2", count=count, offset=off)
        off += 2 * count
        return a
    packed, su, sv = take(k * n * bits // 16), take(k), take(n)
    inner, orig = take(k * n), take(k * n)
    assert off == len(raw)
    return k, n, bits, cb, packed, su, sv, inner.reshape(k, n), orig.reshape(k, n)


@pytest.mark.parametrize("name", ["k4-cb2-128x256.exl3ref", "k3-cb0-128x128.exl3ref"])
def test_exl3ref_fixtures(oracle, name):
    k, n, bits, cb, packed, su, sv, inner, orig = read_exl3ref(GOLD / name)
    assert np.array_equal(oracle.decode_inner(packed, k, n, bits, cb), inner)
    got = oracle.reconstruct(packed, su, sv, k, n, bits, cb).view(np.float16).astype(np.float64)
    ref = orig.view(np.float16).astype(np.float64)
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) <= 0.002     # tools/exl3_verify.cpp:69
    assert np.sum((got - ref) ** 2) / np.sum(ref ** 2) <= 1e-6


def test_model_reader_known_answer(oracle):
    # tests/test_model_reader.cpp:51-56: zero trellis, su = sv = 1 -> column 0 = 128 * code(0) at row 0, zeros elsewhere
    k = n = 128
    packed = np.zeros(k * n * 4 // 16, np.uint16)
    one = np.full(128, 0x3C00, np.uint16)
    w = oracle.reconstruct(packed, one, one, k, n, 4, 2)
    code = oracle.L.orc_half_to_float(oracle.L.orc_decode_codebook(0, 2))
    assert w[0, 0] == oracle.L.orc_float_to_half(code * 128)
    assert np.all(w.view(np.float16).reshape(-1)[1:] == 0)


# ---- GET_ROWS (src/exl3-ggml.cpp:19-49) ---------------------------------------------

def test_get_rows_golden(oracle):
    d = np.load(GOLD / "get_rows.npz")
    k, n, bits, cb, seed = (int(v) for v in d["meta"])
    p = synth.packed_tiles(seed, k, n, bits)
    su, sv = synth.layer_scales(seed, k, n)
    rec = synth.pack_records(p, su, sv, bits).view(np.uint8)
    assert sha(rec) == str(d["records_sha256"])
    got = oracle.get_rows(rec, bits, cb, k, n, d["ids"])
    assert np.array_equal(got.view(np.uint32), d["out"].view(np.uint32))


@pytest.mark.parametrize("bits,cb", [(4, 2), (3, 0), (6, 1)])
def test_get_rows_is_a_reconstruct_column(oracle, bits, cb):
    # each id's row is column id of the whole-matrix reconstruct (su from the record's
    # kb, sv from its nb): catches a wrong record, column or transposition
    k, n = 256, 384
    p = synth.packed_tiles(31 + bits, k, n, bits)
    su, sv = synth.layer_scales(31 + bits, k, n)
    rec = synth.pack_records(p, su, sv, bits).view(np.uint8)
    ids = np.array([0, n // 2, n - 1, 127, 128, 300], dtype=np.int32)
    full = oracle.reconstruct(p, su, sv, k, n, bits, cb).view(np.float16).astype(np.float32)
    got = oracle.get_rows(rec, bits, cb, k, n, ids)
    assert np.array_equal(got, full[:, ids].T)


def test_get_rows_model_reader_known_answer(oracle):
    # tests/test_model_reader.cpp:51-56 through GET_ROWS: zero trellis, su = sv = 1:
    # row 0 = [fp16(128 code(0)), 0, ...], row 1 = zeros (H 1 = sqrt(128) e0)
    k = n = 128
    p = np.zeros((k // 16, n // 16, 16 * 4), np.uint16)
    one = np.ones(128, np.float16)
    rec = synth.pack_records(p, one, one, 4).view(np.uint8)
    got = oracle.get_rows(rec, 4, 2, k, n, np.array([0, 1], np.int32))
    code = oracle.L.orc_half_to_float(oracle.L.orc_decode_codebook(0, 2))
    assert got[0, 0] == np.float16(code * 128) and np.all(got[0, 1:] == 0) and np.all(got[1] == 0)
    with pytest.raises(ValueError):
        oracle.get_rows(rec, 4, 2, k, n, np.array([0, n], np.int32))
    with pytest.raises(ValueError):
        oracle.get_rows(rec, 4, 2, k, n, np.array([-1], np.int32))


# ---- records --------------------------------------------------------------------

def test_pack_records_matches_numpy_and_decodes(oracle):
    k, n, bits = 256, 384, 5
    p = synth.packed_tiles(11, k, n, bits)
    su, sv = synth.layer_scales(11, k, n)
    rec_c = oracle.pack_records(p, su, sv, k, n, bits)
    rec_np = synth.pack_records(p, su, sv, bits).view(np.uint8)
    assert np.array_equal(rec_c, rec_np)
    assert rec_c.nbytes == (k // 128) * (n // 128) * synth.group_bytes(bits)
    for cb in range(3):
        assert np.array_equal(oracle.decode_records(rec_c, k, n, bits, cb), oracle.decode_inner(p, k, n, bits, cb))


def test_validate_records(oracle):
    k, n, bits = 128, 256, 4
    p = synth.packed_tiles(12, k, n, bits)
    su, sv = synth.layer_scales(12, k, n)
    rec = synth.pack_records(p, su, sv, bits).view(np.uint8).copy()
    assert oracle.validate_records(rec, bits) == 1
    bad = rec.copy().view(np.uint16)
    bad[(2048 * bits + 256 + 10) // 2] = 0x7C00  # +inf in sv of record 0
    assert oracle.validate_records(bad.view(np.uint8), bits) == 0
    assert oracle.validate_records(rec[:-2], bits) == -1


# ---- the CPU layer ----------------------------------------------------------------

def layer64(inner_u16, su, sv, x):
    """float64 y = sv * H_n((H_k(x * su)) @ W_hat), the layer of src/exl3-ggml.cpp:51-92"""
    k, n = inner_u16.shape
    H = h128_matrix()
    W = inner_u16.view(np.float16).astype(np.float64)
    xh = (x.astype(np.float64) * su.astype(np.float64)).reshape(-1, k // 128, 128) @ H.T
    acc = xh.reshape(-1, k) @ W
    return (acc.reshape(-1, n // 128, 128) @ H.T).reshape(-1, n) * sv.astype(np.float64)


def nmse(a, b):
    return float(np.sum((a - b) ** 2) / np.sum(b ** 2))


def test_layer_golden(oracle):
    d = np.load(GOLD / "layer.npz", allow_pickle=False)
    k, n, bits, cb, rows = (int(v) for v in d["meta"])
    y = oracle.mul_mat(d["records"], bits, cb, k, n, d["x"])
    assert nmse(y, d["y"]) < 1e-10              # fp32 vs float64 of the same math
    assert nmse(y, d["y_from_reconstruct"]) < 1e-5   # tests/test-exl3-graph.cpp:100-104 gate
    x32 = d["x"].astype(np.float32)
    assert np.array_equal(oracle.mul_mat(d["records"], bits, cb, k, n, x32), y)  # f32 input of fp16 values


@pytest.mark.parametrize("bits,cb", [(2, 2), (3, 0), (6, 1), (8, 2)])
def test_layer_vs_float64(oracle, bits, cb):
    k, n, rows = 384, 256, 4
    p = synth.packed_tiles(bits * 10 + cb, k, n, bits)
    su, sv = synth.layer_scales(7, k, n)
    x = synth.activations(8, rows, k)
    rec = synth.pack_records(p, su, sv, bits)
    y = oracle.mul_mat(rec, bits, cb, k, n, x)
    assert nmse(y, layer64(oracle.decode_inner(p, k, n, bits, cb), su, sv, x)) < 1e-10


def test_layer_thread_partition_bit_identical(oracle):
    k, n, bits = 256, 640, 4
    p = synth.packed_tiles(21, k, n, bits)
    su, sv = synth.layer_scales(21, k, n)
    rec = synth.pack_records(p, su, sv, bits)
    x = synth.activations(22, 3, k)
    y1 = oracle.mul_mat(rec, bits, 2, k, n, x, threads=1)
    for t in (2, 3, 8):
        assert np.array_equal(oracle.mul_mat(rec, bits, 2, k, n, x, threads=t), y1)
    # a bounded sample of column groups equals the same columns of the full run
    ys = oracle.mul_mat(rec, bits, 2, k, n, x, threads=2, groups=(1, 3))
    assert np.array_equal(ys[:, 128:384], y1[:, 128:384])


def upstream_from_records(rec, k, n, bits):
    """Records (u16 view) -> upstream tiles [k/16, n/16, 16 bits], su [k], sv [n] (the inverse of the
    record assembly of tools/export_native_gguf.py:27-36)."""
    recs = rec.reshape(n // 128, k // 128, -1)
    tiles = recs[:, :, : 1024 * bits]
    p = tiles.reshape(n // 128, k // 128, 8, 8, 16 * bits).transpose(1, 2, 0, 3, 4).reshape(k // 16, n // 16, 16 * bits)
    su = recs[0, :, 1024 * bits: 1024 * bits + 128].reshape(-1).view(np.float16)
    sv = recs[:, 0, 1024 * bits + 128:].reshape(-1).view(np.float16)
    return np.ascontiguousarray(p), np.ascontiguousarray(su), np.ascontiguousarray(sv)


def test_iface_matmul_layer_golden(oracle):
    """The DSP service's layer (src/hexagon/exl3_service.c:265-305: upstream tiles, separate su/sv,
    fp32 in and out) on the layer fixture, whose records carry the same tiles and scales."""
    d = np.load(GOLD / "layer.npz", allow_pickle=False)
    k, n, bits, cb, rows = (int(v) for v in d["meta"])
    p, su, sv = upstream_from_records(d["records"], k, n, bits)
    y = oracle.iface_matmul(p, su, sv, bits, cb, k, n, d["x"].astype(np.float32))
    assert nmse(y, d["y"]) < 1e-10
    assert nmse(y, d["y_from_reconstruct"]) < 1e-5   # tests/test-exl3-graph.cpp:100-104 gate


@pytest.mark.parametrize("bits,cb", [(1, 2), (3, 0), (5, 1), (8, 2)])
def test_iface_matmul_vs_float64_and_ggml_layer(oracle, bits, cb):
    k, n, rows = 384, 256, 8
    p = synth.packed_tiles(bits * 17 + cb, k, n, bits)
    su, sv = synth.layer_scales(bits + 40, k, n)
    x = synth.activations(bits + 50, rows, k).astype(np.float32)
    y = oracle.iface_matmul(p, su, sv, bits, cb, k, n, x)
    assert nmse(y, layer64(oracle.decode_inner(p, k, n, bits, cb), su, sv, x)) < 1e-10
    # the ggml op on the records of the same weights: same math, another fp32 summation order
    y_ggml = oracle.mul_mat(synth.pack_records(p, su, sv, bits), bits, cb, k, n, x)
    assert nmse(y, y_ggml) < 1e-11
    # a wrong tile order (column-major tile grid) or swapped scale vectors fail the float64 check
    p_t = np.ascontiguousarray(p.reshape(k // 16, n // 16, -1).transpose(1, 0, 2)).reshape(k // 16, n // 16, -1)
    assert nmse(oracle.iface_matmul(p_t, su, sv, bits, cb, k, n, x), y) > 1e-3
    assert nmse(oracle.iface_matmul(p, su[::-1].copy(), sv, bits, cb, k, n, x), y) > 1e-3


def test_iface_matmul_rejects(oracle):
    """The service's argument checks (src/hexagon/exl3_service.c:270-273)."""
    p = np.zeros(16, dtype=np.uint16)
    s = np.zeros(128, dtype=np.float16)

    def rejects(bits, cb, k, n, batch):
        with pytest.raises(ValueError):
            oracle.iface_matmul(p, s, s, bits, cb, k, n, np.zeros((batch, k), dtype=np.float32))

    rejects(0, 2, 128, 128, 1)
    rejects(9, 2, 128, 128, 1)
    rejects(4, 3, 128, 128, 1)
    rejects(4, 2, 100, 128, 1)
    rejects(4, 2, 128, 96, 1)
    rejects(4, 2, 128, 128, 9)        # batch above 8
    rejects(4, 2, 8192, 8320, 1)      # k * n above 64 Mi
    with pytest.raises(ValueError):
        oracle.iface_matmul(p, s, s, 4, 2, 128, 128, np.zeros((0, 128), dtype=np.float32))


def test_planted_mistakes_fail_the_gate(oracle):
    """The NMSE gate used for the layer catches plausible slips in the formula."""
    d = np.load(GOLD / "layer.npz", allow_pickle=False)
    k, n, bits, cb, rows = (int(v) for v in d["meta"])
    rec, x, y_ref = d["records"], d["x"], d["y_from_reconstruct"]
    p, su, sv = upstream_from_records(rec, k, n, bits)
    inner = oracle.decode_inner(p, k, n, bits, cb)
    good = layer64(inner, su, sv, x)
    assert nmse(good, y_ref) < 1e-5
    H = h128_matrix()
    W = inner.view(np.float16).astype(np.float64)
    mistakes = {
        "dropped su": layer64(inner, np.ones_like(su), sv, x),
        "dropped sv": layer64(inner, su, np.ones_like(sv), x),
        "no output H128": ((x.astype(np.float64) * su).reshape(-1, k // 128, 128) @ H).reshape(-1, k) @ W * sv.astype(np.float64),
        "transposed tiles": layer64(inner.reshape(k // 16, 16, n // 16, 16).transpose(0, 3, 2, 1).reshape(k, n).copy(), su, sv, x),
        "wrong codebook": layer64(oracle.decode_inner(p, k, n, bits, 0), su, sv, x),
        "unscaled H": layer64(inner, su, sv, x) * 128.0,
    }
    for name, bad in mistakes.items():
        assert nmse(bad, y_ref) > 1e-3, name
