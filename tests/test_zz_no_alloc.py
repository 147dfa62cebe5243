"""exl3_hip_mul_mat_noalloc: the layer without a workspace and without
allocation (its workspace is a 64 MiB device array inside the library, one per
GPU).  Checked through the C-ABI against exl3_hip_mul_mat with a fresh caller
workspace, bit for bit (the same kernels and plans), on calls in a row whose
second input is smaller, across kernels (GEMV, GEMM) and shapes; under HIP-graph
capture (which refuses allocation) with replays equal to eager calls; and its
refusals of requests beyond the array."""
import ctypes

import numpy as np
import pytest

import synth
from gpu_util import dev

pytestmark = pytest.mark.gpu


def make_layer(seed, k, n, bits):
    p = synth.packed_tiles(seed, k, n, bits)
    su, sv = synth.layer_scales(seed, k, n)
    return dev(synth.pack_records(p, su, sv, bits).view(np.uint8))


def noalloc(amd, rec, bits, k, n, x, y, stream=None):
    import torch
    st = amd.lib().exl3_hip_mul_mat_noalloc(
        amd._ptr(rec), bits, amd.CB_MUL1, k, n, amd._ptr(x), amd.F16 if x.dtype == torch.float16 else amd.F32,
        x.shape[0], x.stride(0), amd._ptr(y), amd.F16 if y.dtype == torch.float16 else amd.F32, y.stride(0),
        amd._stream(stream))
    return st


def with_workspace(amd, rec, bits, k, n, x, out_dtype):
    import torch
    ws = amd.new_workspace(k, n, x.shape[0])
    y = amd.mul_mat(rec, bits, k, n, x, out_dtype=out_dtype, workspace=ws)
    torch.cuda.synchronize()
    return y


def test_noalloc_matches_mul_mat_on_consecutive_calls(amd):
    import torch
    cases = [  # (k, n, bits, rows) in call order: each second call of a pair is smaller
        (14336, 4096, 4, 8), (14336, 4096, 4, 3),     # GEMV, then a smaller GEMV
        (4096, 2048, 4, 64), (4096, 2048, 4, 1),      # GEMM, then a GEMV on the same array
        (2048, 6144, 3, 24), (2048, 6144, 3, 17),     # GEMM, 32-row tiles
        (1024, 512, 5, 300), (1024, 512, 5, 33),      # two GEMM m-tiles, then one
        (512, 65664, 2, 40), (512, 65664, 2, 2),      # n above 65536: GEMM, then GEMV
    ]
    layers = {}
    for i, (k, n, bits, rows) in enumerate(cases):
        key = (k, n, bits)
        if key not in layers:
            layers[key] = make_layer(2000 + i, k, n, bits)
        rec = layers[key]
        x = torch.from_numpy(synth.activations(2100 + i, rows, k)).cuda()
        for out_dtype in (torch.float16, torch.float32):
            y = torch.full((rows, n), float("nan"), dtype=out_dtype, device="cuda")
            assert noalloc(amd, rec, bits, k, n, x, y) == amd.OK, (k, n, rows)
            torch.cuda.synchronize()
            ref = with_workspace(amd, rec, bits, k, n, x, out_dtype)
            assert torch.equal(y, ref), f"call {i}: k={k} n={n} rows={rows} {out_dtype}"
            print(f"  noalloc call {i}: k={k} n={n} bits={bits} rows={rows} {out_dtype}: equal", flush=True)


def test_noalloc_under_graph_capture(amd):
    """A captured call allocates nothing (global capture mode would fail on an
    allocation); replays with eager work in between equal the eager result."""
    import torch
    k, n, bits, rows = 2048, 4096, 4, 5
    rec = make_layer(2200, k, n, bits)
    x = torch.from_numpy(synth.activations(2201, rows, k)).cuda()
    ref = with_workspace(amd, rec, bits, k, n, x, torch.float16)
    y = torch.empty((rows, n), dtype=torch.float16, device="cuda")
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s, capture_error_mode="global"):
        assert noalloc(amd, rec, bits, k, n, x, y, stream=s) == amd.OK
    for rep in range(3):
        y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ref), f"replay {rep}"
        y2 = torch.empty_like(y)   # an eager call on the same array between replays
        assert noalloc(amd, rec, bits, k, n, x, y2) == amd.OK
        torch.cuda.synchronize()
        assert torch.equal(y2, ref)


def test_noalloc_refuses_beyond_its_array(amd):
    import torch
    x = torch.zeros((1, 128), dtype=torch.float16, device="cuda")
    y = torch.zeros((1, 128), dtype=torch.float16, device="cuda")
    rec = torch.zeros(2048 * 4 + 512, dtype=torch.uint8, device="cuda")
    L = amd.lib()
    # workspace beyond 64 MiB (a 65536-row GEMM at k = 16384): refused before any work
    big = L.exl3_hip_mul_mat_workspace_bytes(16384, 4096, 65536)
    assert big > (64 << 20)
    st = L.exl3_hip_mul_mat_noalloc(amd._ptr(rec), 4, 2, 16384, 4096, amd._ptr(x), amd.F16, 65536, 16384,
                                    amd._ptr(y), amd.F16, 4096, None)
    assert st == amd.WORKSPACE_TOO_SMALL
    # the layer's own argument checks
    assert L.exl3_hip_mul_mat_noalloc(None, 4, 2, 128, 128, amd._ptr(x), amd.F16, 1, 128, amd._ptr(y), amd.F16,
                                      128, None) == amd.INVAL_PARAMS
    assert L.exl3_hip_mul_mat_noalloc(amd._ptr(rec), 9, 2, 128, 128, amd._ptr(x), amd.F16, 1, 128, amd._ptr(y),
                                      amd.F16, 128, None) == amd.INVAL_PARAMS
