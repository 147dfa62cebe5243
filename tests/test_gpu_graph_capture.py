"""HIP graph capture of the entry points other than exl3_hip_mul_mat (whose own
replay test is in test_gpu_layer.py): grouped projections on the GEMV (rows 8)
and on its 17..32-row mode with the separate activation prep (rows 24), the
batched dequantisation and GET_ROWS.  Each graph is replayed several times with
its outputs poisoned before every replay and eager calls on the same workspace
between the replays; every replay must equal the eager result bit for bit.  The
eager results are pinned to the oracle: its restatement of ggml_exl3_mul_mat
(src/exl3-ggml.cpp:51-92) at the layer tolerance, its decode_inner and its
GET_ROWS bit for bit."""
import numpy as np
import pytest

import synth
from gpu_util import assert_layer_close, dev, host_u16

pytestmark = pytest.mark.gpu
THREADS = 8
MUL1 = 2


def make_layer(seed, k, n, bits):
    p = synth.packed_tiles(seed, k, n, bits)
    su, sv = synth.layer_scales(seed, k, n)
    return synth.pack_records(p, su, sv, bits).view(np.uint8)


@pytest.mark.parametrize("rows", [8, 24])
def test_group_graph_replay(amd, oracle, rows):
    import torch
    k = 2048
    qkv = [(2048, 6), (512, 6), (512, 6)]        # q/k/v of one layer: one grouped launch
    gu = [(6144, 4), (6144, 4)]                  # gate/up
    recs_h = [make_layer(1200 + i, k, n, b) for i, (n, b) in enumerate(qkv + gu)]
    recs = [dev(r) for r in recs_h]
    x = torch.from_numpy(synth.activations(1300 + rows, rows, k)).cuda()
    need = max(amd.group_workspace_bytes(k, [n for n, _ in qkv], rows),
               amd.group_workspace_bytes(k, [n for n, _ in gu], rows), amd.workspace_bytes(k, 2048, rows))
    ws = amd.new_workspace(k, 2048, rows, nbytes=need)
    ys = [torch.empty((rows, n), dtype=torch.float32, device="cuda") for n, _ in qkv + gu]

    def calls():
        amd.mul_mat_group([(recs[i], qkv[i][0], ys[i]) for i in range(3)], 6, k, x, codebook=MUL1, workspace=ws)
        amd.mul_mat_group([(recs[3 + i], gu[i][0], ys[3 + i]) for i in range(2)], 4, k, x, codebook=MUL1,
                          workspace=ws)

    calls()
    torch.cuda.synchronize()
    eager = [y.clone() for y in ys]
    for i, (n, bits) in enumerate(qkv + gu):
        want = oracle.mul_mat(recs_h[i], bits, MUL1, k, n, x.cpu().numpy(), threads=THREADS)
        assert_layer_close(eager[i].cpu().numpy(), want, what=f"group matrix {i} rows={rows}")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        calls()
    for rep in range(4):
        print(f"  group graph rows={rows} replay {rep}", flush=True)
        for y in ys:
            y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for i, y in enumerate(ys):
            assert torch.equal(y, eager[i]), f"replay {rep} matrix {i} rows={rows}"
        # eager work on the same workspace between replays: a plain call of another shape
        amd.mul_mat(recs[0], 6, k, 2048, x, codebook=MUL1, workspace=ws)
        torch.cuda.synchronize()


def test_decode_batch_graph_replay(amd, oracle):
    import torch
    gen = torch.Generator(device="cuda")
    shapes = [(128, 256, 3), (256, 128, 6), (2048, 512, 4), (512, 2048, 2), (384, 640, 5), (128, 128, 8)]
    items = []
    for j, (k, n, bits) in enumerate(shapes):
        gen.manual_seed(900 + j)
        p = torch.randint(-32768, 32768, (k * n * bits // 16,), generator=gen, device="cuda",
                          dtype=torch.int32).to(torch.int16)
        items.append((p, bits, k, n, torch.empty((k, n), dtype=torch.int16, device="cuda")))
    outs = amd.decode_batch(items, codebook=MUL1)
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs]
    for (p, bits, k, n, _), e in zip(items, eager):
        if k * n <= 128 * 256:
            want = oracle.decode_inner(p.cpu().numpy().view(np.uint16), k, n, bits, MUL1)
            assert np.array_equal(host_u16(e), want), (bits, k, n)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        amd.decode_batch(items, codebook=MUL1)
    for rep in range(3):
        print(f"  decode_batch graph replay {rep}", flush=True)
        for o in outs:
            o.fill_(-1)
        g.replay()
        torch.cuda.synchronize()
        for j, (o, e) in enumerate(zip(outs, eager)):
            assert torch.equal(o, e), f"replay {rep} matrix {j}"
        amd.decode(items[2][0], 4, 2048, 512, codebook=MUL1)  # eager work between replays
        torch.cuda.synchronize()


def test_get_rows_graph_replay(amd, oracle):
    import torch
    k, n, bits = 2048, 1024, 6
    rec_h = make_layer(1400, k, n, bits)
    rec = dev(rec_h)
    ids_h = np.array([0, 5, 1023, 77, 512, 5, 300, 999], dtype=np.int32)
    ids = torch.from_numpy(ids_h).cuda()
    out = torch.empty((len(ids_h), k), dtype=torch.float32, device="cuda")
    amd.get_rows(rec, bits, k, n, ids, codebook=MUL1, out=out)
    torch.cuda.synchronize()
    eager = out.clone()
    want = oracle.get_rows(rec_h, bits, MUL1, k, n, ids_h)
    assert np.array_equal(eager.cpu().numpy().view(np.uint32), want.view(np.uint32))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        amd.get_rows(rec, bits, k, n, ids, codebook=MUL1, out=out)
    for rep in range(3):
        print(f"  get_rows graph replay {rep}", flush=True)
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep}"
