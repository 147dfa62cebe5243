"""The reference's on-device layer matrix on this path.

The reference runs its graph test (tests/test-exl3-graph.cpp: MUL_MAT followed
by a residual ADD, gated at NMSE < 1e-5 against float64 x . W_original +
residual, :51-55, :89-104) as 84 cases: 4/6/8 bits x f32/f16 input x batch
1/4/8/32/37/128/512 x two Hexagon backends
(docs/validation/packed-rounding-optimization.md:12).  Here the same bits,
input types and batches run through exl3_hip_mul_mat_add on the 256 x 384 mul1
matrices of the reference fixture geometry (tests/generate_cuda_fixtures.py:
69-90, seed bits * 100 + codebook, the recipe of matrices.json).  Their
original-basis weights come from this library's reconstruct and must match the
reference's reconstruct digest bit for bit before they serve as the float64
expectation.  The batches reach every launch path at k = 256: the GEMV (1, 4,
8) and the GEMM's 32-, 64-, 128- and 512-row tiles with k split in two records
(32, 37, 128, 512).
"""
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

import synth
from gpu_util import dev, host_u16
from test_oracle import golden_matrix_inputs

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"
MUL1 = 2


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


_weights = {}


def layer(amd, bits):
    """Records and the reference-pinned original-basis weights (float64 [k][n])."""
    if bits not in _weights:
        m = next(m for m in json.loads((GOLD / "matrices.json").read_text()) if m["bits"] == bits and m["cb"] == MUL1)
        p, su, sv = golden_matrix_inputs(m)
        k, n = m["k"], m["n"]
        dp, dsu, dsv = dev(p), dev(su.view(np.uint16)), dev(sv.view(np.uint16))
        orig = host_u16(amd.reconstruct(dp, bits, k, n, su=dsu, sv=dsv, codebook=MUL1))
        assert sha(orig.astype("<u2")) == m["original_sha256"], "reconstruct differs from the reference's"
        rec = amd.pack_records(dp, dsu, dsv, bits, k, n)
        _weights[bits] = (rec, k, n, orig.view(np.float16).astype(np.float64))
    return _weights[bits]


@pytest.mark.parametrize("batch", [1, 4, 8, 32, 37, 128, 512])
@pytest.mark.parametrize("xname", ["f32", "f16"])
@pytest.mark.parametrize("bits", [4, 6, 8])
def test_graph_matrix(amd, bits, xname, batch):
    import torch
    rec, k, n, w = layer(amd, bits)
    # tests/test-exl3-graph.cpp:68-72: deterministic input and residual recipes
    x = (((np.arange(batch * k) * 13) % 17).astype(np.float64) - 8) / 17
    x = x.astype(np.float32).reshape(batch, k)
    if xname == "f16":
        x = x.astype(np.float16)
    residual = (((np.arange(batch * n) % 23).astype(np.float64) - 11) / 7).astype(np.float32).reshape(batch, n)
    y = amd.mul_mat(rec, bits, k, n, torch.from_numpy(np.ascontiguousarray(x)).cuda(), codebook=MUL1,
                    residual=torch.from_numpy(residual).cuda())
    torch.cuda.synchronize()
    actual = y.cpu().numpy().astype(np.float64)
    expected = residual.astype(np.float64) + x.astype(np.float64) @ w
    nmse = np.sum((actual - expected) ** 2) / np.sum(expected ** 2)
    print(f"  bits {bits} input {xname} batch {batch}: nmse={nmse:.2e}", flush=True)
    assert np.all(np.isfinite(actual)) and nmse < 1e-5
    # without the residual the same call gives the layer alone, at the same gate
    plain = amd.mul_mat(rec, bits, k, n, torch.from_numpy(np.ascontiguousarray(x)).cuda(), codebook=MUL1)
    torch.cuda.synchronize()
    lay = plain.cpu().numpy().astype(np.float64)
    ref = x.astype(np.float64) @ w
    assert np.sum((lay - ref) ** 2) / np.sum(ref ** 2) < 1e-5
