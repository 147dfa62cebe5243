"""The layer and GET_ROWS at the size limits.  The reference's device op accepts
k up to 65,536 and n up to 1,048,576 and works through a call's rows in chunks
of at most 1,024 (patches/llama-exl3.patch:185-199, src/exl3-htp.c:165-171);
this library takes up to 65,536 rows in one call and refuses more.  Each case
runs against the oracle's restatement of ggml_exl3_mul_mat
(src/exl3-ggml.cpp:51-92) at the layer tolerance, and GET_ROWS
(src/exl3-ggml.cpp:19-49) bit for bit."""
import numpy as np
import pytest

import synth
from gpu_util import assert_layer_close, dev

pytestmark = pytest.mark.gpu
THREADS = 8
MUL1 = 2


def make_layer(seed, k, n, bits):
    p = synth.packed_tiles(seed, k, n, bits)
    su, sv = synth.layer_scales(seed, k, n)
    return synth.pack_records(p, su, sv, bits).view(np.uint8)


def run(amd, rec_d, bits, k, n, x, cb=MUL1):
    import torch
    y = amd.mul_mat(rec_d, bits, k, n, torch.from_numpy(np.ascontiguousarray(x)).cuda(), codebook=cb)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def test_largest_k(amd, oracle):
    """k = 65,536 (512 records per column group): the GEMV with 256 k-splits of
    two records, and the GEMM's 64- and 256-row tiles with their k splits."""
    k, n, bits = 65536, 256, 4
    rec = make_layer(2100, k, n, bits)
    rd = dev(rec)
    for rows in (1, 8, 40, 130):
        print(f"  k={k} n={n} rows={rows}", flush=True)
        x = synth.activations(2110 + rows, rows, k)
        ref = oracle.mul_mat(rec, bits, MUL1, k, n, x, threads=THREADS)
        assert_layer_close(run(amd, rd, bits, k, n, x), ref, what=f"k={k} rows={rows}")


def test_largest_n(amd, oracle):
    """n = 1,048,576 (8,192 column groups of one record each at k = 128): the
    GEMV without a k split, and the 128-row GEMM tile, which cannot split one
    record; then GET_ROWS of the first, last and scattered columns."""
    import torch
    k, n, bits = 128, 1048576, 2
    rec = make_layer(2200, k, n, bits)
    rd = dev(rec)
    for rows in (1, 3, 40):
        print(f"  k={k} n={n} rows={rows}", flush=True)
        x = synth.activations(2210 + rows, rows, k)
        ref = oracle.mul_mat(rec, bits, MUL1, k, n, x, threads=THREADS)
        assert_layer_close(run(amd, rd, bits, k, n, x), ref, what=f"n={n} rows={rows}")
    ids = np.array([0, n - 1, n // 2, 12345, 777777, n - 128, 1, n - 2], dtype=np.int32)
    got = amd.get_rows(rd, bits, k, n, torch.from_numpy(ids).cuda(), codebook=MUL1).cpu().numpy()
    want = oracle.get_rows(rec, bits, MUL1, k, n, ids)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_rows_beyond_the_reference_chunk_and_at_the_limit(amd, oracle):
    """1,500 rows in one call (the reference's op would chunk them by 1,024) and
    the 65,536 rows this library takes at most; 65,537 are refused."""
    import torch
    for k, n, bits, rows in [(256, 384, 3, 1500), (128, 128, 5, 65536)]:
        print(f"  k={k} n={n} rows={rows}", flush=True)
        rec = make_layer(2300 + bits, k, n, bits)
        x = synth.activations(2310 + bits, rows, k)
        ref = oracle.mul_mat(rec, bits, MUL1, k, n, x, threads=THREADS)
        assert_layer_close(run(amd, dev(rec), bits, k, n, x), ref, what=f"k={k} n={n} rows={rows}")
    rec = dev(make_layer(2320, 128, 128, 4))
    x = torch.zeros((65537, 128), dtype=torch.float16, device="cuda")
    with pytest.raises(amd.Exl3Error) as e:
        amd.mul_mat(rec, 4, 128, 128, x, codebook=MUL1)
    assert e.value.status == amd.INVAL_PARAMS


def test_decode_at_the_limits(amd, oracle):
    """exl3_hip_decode and exl3_hip_decode_batch of the largest k and the largest
    n, bit for bit against the oracle's decode_inner (src/exl3_codec.cpp:117-145)."""
    import torch
    for k, n, bits in [(65536, 256, 5), (128, 1048576, 3)]:
        print(f"  decode k={k} n={n} bits={bits}", flush=True)
        p = synth.packed_tiles(2400 + bits, k, n, bits)
        pd = dev(p)
        want = oracle.decode_inner(p, k, n, bits, MUL1)
        got = amd.decode(pd, bits, k, n, codebook=MUL1)
        torch.cuda.synchronize()
        assert np.array_equal(got.cpu().numpy().view(np.uint16), want)
        (batch,) = amd.decode_batch([(pd, bits, k, n, None)], codebook=MUL1)
        torch.cuda.synchronize()
        assert torch.equal(batch, got)
