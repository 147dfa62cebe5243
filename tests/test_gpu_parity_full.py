"""Full-size parity where sampled checks used to stand in:

* the M=512 prefill GEMM (k=14336 in, n=4096 out, 4 bits) on all 512 rows, and
  the GEMM at the 33..128-row counts of continuous-batching prefill chunks,
  against a float64 evaluation of the layer on the oracle's decoded weights
  (the layer of src/exl3-ggml.cpp:51-92); tolerance max-abs 1e-2, rel-L2 1e-3;
* the dequant sweep over the 151 matrices of the 2B hybrid model, decoded by
  one exl3_hip_decode_batch call as the bench times it, bit for bit against
  the oracle's decode_inner of every matrix, the full 2048 x 151,936 6-bit
  vocabulary head included."""
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import synth
from gpu_util import assert_layer_close, dev
from test_oracle import layer64

pytestmark = pytest.mark.gpu


def oracle_decode(oracle, p, k, n, bits, cb, threads=16):
    """decode_inner in column slices on several threads (ctypes drops the GIL)"""
    width = max(16, (n // threads + 15) // 16 * 16)
    out = np.empty((k, n), dtype=np.uint16)

    def part(first):
        cnt = min(width, n - first)
        out[:, first:first + cnt] = oracle.decode_inner(p, k, n, bits, cb, first=first, count=cnt)
    with ThreadPoolExecutor(threads) as ex:
        list(ex.map(part, range(0, n, width)))
    return out


@pytest.fixture(scope="module")
def c3_layer(oracle):
    k, n, bits = 14336, 4096, 4
    p = synth.packed_tiles(1505, k, n, bits)
    su, sv = synth.layer_scales(1505, k, n)
    rec = synth.pack_records(p, su, sv, bits).view(np.uint8)
    return k, n, bits, dev(rec), oracle_decode(oracle, p, k, n, bits, 2), su, sv


@pytest.mark.parametrize("rows", [512, 33, 48, 64, 96, 128])
def test_gemm_full_size_all_rows_vs_float64(amd, c3_layer, rows):
    import torch
    k, n, bits, rd, inner, su, sv = c3_layer
    x = synth.activations(1600 + rows, rows, k)
    y = amd.mul_mat(rd, bits, k, n, torch.from_numpy(x).cuda(), out_dtype=torch.float16)
    torch.cuda.synchronize()
    ref = layer64(inner, su, sv, x.astype(np.float64))
    assert_layer_close(y.float().cpu().numpy(), ref, what=f"k=14336 n=4096 rows={rows} (all rows) vs float64")


def test_dequant_sweep_151_matrices_bit_exact(amd, oracle):
    import torch
    mats = synth.c2_matrices()
    bits = synth.c2_bits(mats)
    packed = [synth.packed_tiles(9100 + i, k, n, int(b)) for i, ((k, n), b) in enumerate(zip(mats, bits))]
    offs = [0]
    for k, n in mats:
        offs.append(offs[-1] + ((k * n + 63) // 64) * 64)
    dst = torch.empty(offs[-1], dtype=torch.int16, device="cuda")
    outs = [dst[o: o + k * n].view(k, n) for o, (k, n) in zip(offs, mats)]
    srcs = [dev(p) for p in packed]
    amd.decode_batch([(s, int(b), k, n, o) for s, b, (k, n), o in zip(srcs, bits, mats, outs)], codebook=2)
    torch.cuda.synchronize()
    print(f"  decoded {len(mats)} matrices, {sum(k * n for k, n in mats)} weights, mean "
          f"{sum(k * n * int(b) for (k, n), b in zip(mats, bits)) / sum(k * n for k, n in mats):.3f} bpw", flush=True)
    for i, ((k, n), b) in enumerate(zip(mats, bits)):
        got = outs[i].cpu().numpy().view(np.uint16)
        want = oracle_decode(oracle, packed[i], k, n, int(b), 2)
        assert np.array_equal(got, want), f"matrix {i} ({k}x{n}, {b} bits)"
    assert mats[-1] == (2048, 151936)   # the full vocabulary head was among them


def test_vocabulary_head_6bit_bit_exact(amd, oracle):
    """The 2B model's tied vocabulary head at its deployed rate, 6 bits
    (k=2048 hidden, n=151,936 vocabulary), decoded whole from upstream tiles and
    from group records: every fp16 weight equals the oracle's decode_inner."""
    import torch
    k, n, bits = 2048, 151936, 6
    p = synth.packed_tiles(9300, k, n, bits)
    want = oracle_decode(oracle, p, k, n, bits, 2)
    got = amd.decode(dev(p), bits, k, n, codebook=2).cpu().numpy().view(np.uint16)
    assert np.array_equal(got, want), "upstream tiles"
    su, sv = synth.layer_scales(9300, k, n)
    rec = synth.pack_records(p, su, sv, bits).view(np.uint8)
    got = amd.decode(dev(rec), bits, k, n, codebook=2, layout=amd.LAYOUT_RECORDS).cpu().numpy().view(np.uint16)
    torch.cuda.synchronize()
    assert np.array_equal(got, want), "records"
