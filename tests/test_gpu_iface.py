"""GPU parity of exl3_hip_iface_matmul, the DSP service's layer
(src/hexagon/exl3_service.c:265-305): upstream tiles with separate su/sv, fp32 in
and out, against the oracle's restatement of that service.  Tolerance: max-abs
<= 1e-2 and relative L2 <= 1e-3 (the layer bar); against exl3_hip_mul_mat on
records packed from the same weights the result is bit-identical (same kernels)."""
import numpy as np
import pytest

import synth
from gpu_util import assert_layer_close, dev

pytestmark = pytest.mark.gpu


def upstream(seed, k, n, bits):
    p = synth.packed_tiles(seed, k, n, bits)
    su, sv = synth.layer_scales(seed, k, n)
    return p, su, sv


@pytest.mark.parametrize("bits,cb,rows", [(4, 2, 1), (4, 2, 8), (2, 0, 3), (6, 1, 5), (3, 2, 12), (5, 2, 40)])
def test_iface_matmul_matches_service_restatement(amd, oracle, bits, cb, rows):
    import torch
    k, n = 512, 384
    p, su, sv = upstream(600 + bits * 7 + rows, k, n, bits)
    x = synth.activations(700 + rows, rows, k).astype(np.float32)
    print(f"  iface_matmul k={k} n={n} bits={bits} cb={cb} rows={rows}", flush=True)
    pd, sud, svd, xd = dev(p), dev(su.view(np.uint16)), dev(sv.view(np.uint16)), torch.from_numpy(x).cuda()
    y = amd.iface_matmul(pd, sud, svd, xd, bits, k, n, codebook=cb)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    if rows <= 8:  # the service's own batch limit
        ref = oracle.iface_matmul(p, su, sv, bits, cb, k, n, x)
    else:          # beyond it the ggml op on the records of the same weights is the reference
        ref = oracle.mul_mat(synth.pack_records(p, su, sv, bits), bits, cb, k, n, x)
    assert_layer_close(y, ref, what=f"iface bits={bits} cb={cb} rows={rows}")
    # the same kernels as exl3_hip_mul_mat on records packed from these weights
    rec = amd.pack_records(pd, sud, svd, bits, k, n)
    y2 = amd.mul_mat(rec, bits, k, n, xd, codebook=cb, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert np.array_equal(y, y2.cpu().numpy())


def test_iface_matmul_caller_workspace_repeated_calls(amd, oracle):
    """A caller workspace serves calls of any batch up to its size, back to back (the split-K
    counters reset themselves), and the result does not depend on which workspace is used."""
    import torch
    k, n, bits = 1024, 512, 4
    p, su, sv = upstream(650, k, n, bits)
    pd, sud, svd = dev(p), dev(su.view(np.uint16)), dev(sv.view(np.uint16))
    ws = amd.new_iface_workspace(bits, k, n, 8)
    for rows in (8, 1, 3, 8):
        x = synth.activations(660 + rows, rows, k).astype(np.float32)
        print(f"  iface_matmul workspace k={k} n={n} rows={rows}", flush=True)
        xd = torch.from_numpy(x).cuda()
        y = amd.iface_matmul(pd, sud, svd, xd, bits, k, n, workspace=ws)
        y_int = amd.iface_matmul(pd, sud, svd, xd, bits, k, n)
        torch.cuda.synchronize()
        y = y.cpu().numpy()
        assert np.array_equal(y, y_int.cpu().numpy())
        assert_layer_close(y, oracle.iface_matmul(p, su, sv, bits, 2, k, n, x), what=f"rows={rows}")
    small = ws[: ws.numel() - 1]
    with pytest.raises(amd.Exl3Error):
        amd.iface_matmul(pd, sud, svd, torch.zeros((8, k), device="cuda"), bits, k, n, workspace=small)
