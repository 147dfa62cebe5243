"""The split-K hand-off's failure path (include/exl3_hip.h: exl3_hip_workspace_status).
A failure is forced from the host with the library's test hook: the workgroups of k
split 0 skip storing their partial and the wait budget is 64 polls, so the summing
workgroups' own bounded wait runs out and every kernel ends normally.  Checked: every
output is NaN (each output column's H128 needs split 0's partial), the workspace's
status word is set, the next call with that workspace (no injection) is NaN again
without waiting, and exl3_hip_workspace_init restores results bit-identical to a
clean run.  GEMV modes: rows 1 (one block), 12 (two blocks, hi/lo), 20 (grouped call,
activations prepared once); a caller workspace and the internal one."""
import numpy as np
import pytest

import synth
from gpu_util import dev

pytestmark = pytest.mark.gpu


def make_layer(seed, k, n, bits):
    p = synth.packed_tiles(seed, k, n, bits)
    su, sv = synth.layer_scales(seed, k, n)
    return dev(synth.pack_records(p, su, sv, bits).view(np.uint8))


def call(amd, rows, rec, bits, k, n, x, ws):
    if rows <= 14:
        return [amd.mul_mat(rec, bits, k, n, x, workspace=ws)]
    return amd.mul_mat_group([(rec, n), (rec, n)], bits, k, x, workspace=ws)


def injected(amd, fn):
    amd.lib().exl3_hip_test_exchange_fault(64, 0)
    try:
        return fn()
    finally:
        amd.lib().exl3_hip_test_exchange_fault(0, -1)


@pytest.mark.parametrize("rows,internal", [(1, False), (12, False), (20, False), (1, True)])
def test_give_up_is_loud_sticky_and_recoverable(amd, rows, internal):
    import torch
    k, n, bits = 2048, 1024, 4   # 8 column groups (16 for the grouped call) x 16 k splits
    print(f"  exchange fault rows={rows} internal={internal}", flush=True)
    rec = make_layer(41, k, n, bits)
    x = torch.from_numpy(synth.activations(42 + rows, rows, k)).cuda()
    ws = None
    if not internal:
        ws = torch.empty(amd.group_workspace_bytes(k, [n, n], rows), dtype=torch.uint8, device="cuda")
        amd.workspace_init(ws)
    clean = [y.clone() for y in call(amd, rows, rec, bits, k, n, x, ws)]
    torch.cuda.synchronize()
    assert not amd.workspace_faulted(ws)
    assert all(torch.isfinite(y).all() for y in clean)

    ys = injected(amd, lambda: call(amd, rows, rec, bits, k, n, x, ws))
    torch.cuda.synchronize()
    assert all(torch.isnan(y).all() for y in ys), "a partial that never arrived must give NaN"
    assert amd.workspace_faulted(ws), "the give-up must set the workspace's status word"

    ys = call(amd, rows, rec, bits, k, n, x, ws)   # no injection: still loud
    torch.cuda.synchronize()
    assert all(torch.isnan(y).all() for y in ys), "a workspace marked failed must keep giving NaN"
    assert amd.workspace_faulted(ws)

    amd.workspace_init(ws)
    assert not amd.workspace_faulted(ws)
    for _ in range(2):
        ys = call(amd, rows, rec, bits, k, n, x, ws)
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(ys, clean)), "results after re-initialisation"
    assert not amd.workspace_faulted(ws)
