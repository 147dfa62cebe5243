"""Helpers shared by the GPU tests (device upload, tolerance checks)."""
import numpy as np


def dev(a):
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a.copy()).cuda()


def host_u16(t):
    return t.cpu().numpy().view(np.uint16)


def layer_stats(y_gpu, y_ref):
    y = np.asarray(y_gpu, dtype=np.float64)
    r = np.asarray(y_ref, dtype=np.float64)
    err = y - r
    return float(np.max(np.abs(err))), float(np.sqrt(np.sum(err ** 2) / np.sum(r ** 2)))


# Layer tolerance of the layer output against the CPU reference layer:
# max-abs error <= 1e-2 and relative L2 error <= 1e-3 (on fp16 or fp32 outputs).
MAX_ABS = 1e-2
REL_L2 = 1e-3


def assert_layer_close(y_gpu, y_ref, max_abs=MAX_ABS, rel_l2=REL_L2, what=""):
    ma, rl = layer_stats(y_gpu, y_ref)
    print(f"  parity {what}: max_abs={ma:.3e} rel_l2={rl:.3e}", flush=True)
    assert np.all(np.isfinite(np.asarray(y_gpu))), what
    assert ma <= max_abs and rl <= rel_l2, (what, ma, rl)
    return ma, rl
