"""Seeded random sweep of the layer against the oracle: shapes, rates,
codebooks, row counts on both sides of the GEMV/GEMM switch, fp16/fp32
activations and outputs, padded row strides and the fused residual.  Each case
is small enough for the oracle's threaded restatement of ggml_exl3_mul_mat
(src/exl3-ggml.cpp:51-92) to finish in well under a second.  Tolerance:
max-abs <= 1e-2 and relative L2 <= 1e-3, as for every layer test."""
import numpy as np
import pytest

import synth
from gpu_util import assert_layer_close, dev

pytestmark = pytest.mark.gpu
CASES = 48  # 0..35 over all row counts, 36..47 around the kernel boundaries (14 | 15, 32 | 33, 64)
BOUNDARY_ROWS = [14, 15, 16, 17, 24, 32, 33, 48, 64]


def case(i):
    rng = np.random.default_rng(20261202 + i)
    k = 128 * int(rng.integers(1, 25))
    n = 128 * int(rng.integers(1, 13))
    bits = int(rng.integers(1, 9))
    cb = int(rng.integers(0, 3))
    rows = int(rng.choice([1, 2, 3, 5, 7, 8, 9, 13, 31, 64, 129, 257] if i < 36 else BOUNDARY_ROWS))
    while k * n * rows > 40_000_000:
        rows = max(1, rows // 2)
    x16 = bool(rng.integers(0, 2))
    y16 = bool(rng.integers(0, 2))
    pad_x = int(rng.integers(0, 3)) * 8
    pad_y = int(rng.integers(0, 3)) * 8
    residual = bool(rng.integers(0, 3) == 0)
    return k, n, bits, cb, rows, x16, y16, pad_x, pad_y, residual


@pytest.mark.parametrize("i", range(CASES))
def test_random_layer(amd, oracle, i):
    import torch
    k, n, bits, cb, rows, x16, y16, pad_x, pad_y, residual = case(i)
    what = (f"case {i}: k={k} n={n} bits={bits} cb={cb} rows={rows} x{'16' if x16 else '32'} "
            f"y{'16' if y16 else '32'} pads {pad_x}/{pad_y} residual={residual}")
    print(f"  {what}", flush=True)
    p = synth.packed_tiles(3000 + i, k, n, bits)
    su, sv = synth.layer_scales(3000 + i, k, n)
    rec = synth.pack_records(p, su, sv, bits).view(np.uint8)
    x = synth.activations(3100 + i, rows, k)
    xt = x if x16 else x.astype(np.float32)
    xbuf = torch.zeros((rows, k + pad_x), dtype=torch.float16 if x16 else torch.float32, device="cuda")
    xbuf[:, :k] = torch.from_numpy(xt).cuda()
    ydt = torch.float16 if y16 else torch.float32
    ybuf = torch.zeros((rows, n + pad_y), dtype=ydt, device="cuda")
    y = ybuf[:, :n]
    want = oracle.mul_mat(rec, bits, cb, k, n, xt, threads=8)
    kw = {}
    if residual:
        r = synth.activations(3200 + i, rows, n).astype(np.float32)
        rd = torch.from_numpy(r).cuda().to(ydt)
        want = want + rd.float().cpu().numpy()
        kw["residual"] = rd
    amd.mul_mat(dev(rec), bits, k, n, xbuf[:, :k], codebook=cb, y=y, **kw)
    torch.cuda.synchronize()
    assert torch.all(ybuf[:, n:] == 0), "write past the row's n outputs"
    assert_layer_close(y.float().cpu().numpy(), want, what=what)
