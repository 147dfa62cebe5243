"""Fused residual add (exl3_hip_mul_mat_add): y = residual + layer(x).

The reference's graph test builds ADD(MUL_MAT(w, x), residual) and gates it at
NMSE < 1e-5 against float64 x . W_original + residual, with the deterministic
recipes x[i] = ((13 i) % 17 - 8) / 17 and residual[i] = (i % 23 - 11) / 7
(tests/test-exl3-graph.cpp:53-55, 68-72, 89-103); the first test repeats that
check on the reference's own EXL3REF1 fixture.  The others pin the fusion
exactly: the fused call returns the plain call's fp32 result plus the residual,
rounded once to the output dtype, also in place (residual is y)."""
from pathlib import Path

import numpy as np
import pytest

import synth
from gpu_util import dev
from test_oracle import read_exl3ref

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"


def make_layer(seed, k, n, bits):
    p = synth.packed_tiles(seed, k, n, bits)
    su, sv = synth.layer_scales(seed, k, n)
    return synth.pack_records(p, su, sv, bits).view(np.uint8)


@pytest.mark.parametrize("batch", [1, 3, 17, 64])
@pytest.mark.parametrize("xname", ["f32", "f16"])
def test_graph_matmul_add_semantics(amd, oracle, batch, xname):
    import torch
    k, n, bits, cb, packed, su, sv, inner, orig = read_exl3ref(GOLD / "k4-cb2-128x256.exl3ref")
    rec = dev(oracle.pack_records(packed, su, sv, k, n, bits))
    x = (((np.arange(batch * k) * 13) % 17).astype(np.float64) - 8) / 17
    x = x.astype(np.float32)
    if xname == "f16":
        x = x.astype(np.float16)
    residual = (((np.arange(batch * n) % 23).astype(np.float64) - 11) / 7).astype(np.float32).reshape(batch, n)
    xd = torch.from_numpy(np.ascontiguousarray(x.reshape(batch, k))).cuda()
    rd = torch.from_numpy(residual).cuda()
    y = amd.mul_mat(rec, bits, k, n, xd, codebook=cb, residual=rd)
    torch.cuda.synchronize()
    actual = y.cpu().numpy().astype(np.float64)
    w = orig.view(np.float16).astype(np.float64)  # original-basis weights W[k][n]
    expected = residual.astype(np.float64) + x.reshape(batch, k).astype(np.float64) @ w
    nmse = np.sum((actual - expected) ** 2) / np.sum(expected ** 2)
    print(f"  batch {batch} input {xname}: matmul_add_nmse={nmse:.2e}", flush=True)
    assert np.isfinite(nmse) and nmse < 1e-5


@pytest.mark.parametrize("rows", [1, 5, 8, 9, 20, 37, 300])
def test_fused_add_is_plain_result_plus_residual(amd, rows):
    import torch
    k, n, bits = 1024, 384, 4
    rec = dev(make_layer(700 + rows, k, n, bits))
    x = torch.from_numpy(synth.activations(710 + rows, rows, k)).cuda()
    plain = amd.mul_mat(rec, bits, k, n, x)                      # fp32 layer result
    r32 = torch.from_numpy(synth.activations(720 + rows, rows, n).astype(np.float32)).cuda()
    r16 = r32.half()
    y32 = amd.mul_mat(rec, bits, k, n, x, residual=r32)
    y16 = amd.mul_mat(rec, bits, k, n, x, residual=r16)
    inplace = r16.clone()
    amd.mul_mat(rec, bits, k, n, x, y=inplace, residual=inplace)
    torch.cuda.synchronize()
    p = plain.cpu().numpy()
    want32 = p + r32.cpu().numpy()                              # one fp32 rounding
    want16 = (p + r16.cpu().numpy().astype(np.float32)).astype(np.float16)
    assert np.array_equal(y32.cpu().numpy().view(np.uint32), want32.view(np.uint32))
    assert np.array_equal(y16.cpu().numpy().view(np.uint16), want16.view(np.uint16))
    assert np.array_equal(inplace.cpu().numpy().view(np.uint16), want16.view(np.uint16))


def test_residual_strides_and_rejections(amd):
    import torch
    k, n, bits, rows = 256, 256, 3, 3
    rec = dev(make_layer(731, k, n, bits))
    x = torch.from_numpy(synth.activations(732, rows, k)).cuda()
    plain = amd.mul_mat(rec, bits, k, n, x)
    big = torch.from_numpy(synth.activations(733, rows, 2 * n).astype(np.float32)).cuda()
    res = big[:, 64:64 + n]                                      # row stride 2n
    y = torch.empty((rows, n + 128), dtype=torch.float32, device="cuda")[:, :n]
    amd.mul_mat(rec, bits, k, n, x, y=y, residual=res)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), plain.cpu().numpy() + res.cpu().numpy())
    # a residual that overlaps y without being y, or is y with another stride: rejected
    buf = torch.zeros((rows + 1) * n, dtype=torch.float32, device="cuda")
    yv, rv = buf[:rows * n].view(rows, n), buf[64:64 + rows * n].view(rows, n)
    with pytest.raises(amd.Exl3Error):
        amd.mul_mat(rec, bits, k, n, x, y=yv, residual=rv)
    wide = torch.zeros((rows, 2 * n), dtype=torch.float32, device="cuda")
    y2 = wide.view(-1)[:rows * n].view(rows, n)
    with pytest.raises(amd.Exl3Error):
        amd.mul_mat(rec, bits, k, n, x, y=y2, residual=wide[:, :n])  # same start, stride 2n vs n
    torch.cuda.synchronize()
