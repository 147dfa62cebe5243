"""GPU parity of the ggml-view entry points (exl3_hip_mul_mat_nd, exl3_hip_get_rows_nd)
on strided, sliced and permuted 3-D views.  The expectation is built the way the
reference's op addresses rows (src/exl3-ggml.cpp:11-17, 34-36, 64, 88): every row is
gathered from its byte offset i1 nb[1] + i2 nb[2] + i3 nb[3], the oracle's layer (or
GET_ROWS) runs on the gathered rows, and each result row is compared with the bytes at
the same offset of the output view.  Layer tolerance: max-abs <= 1e-2 and relative L2
<= 1e-3; GET_ROWS bit-exact.  Bytes of the output buffers outside the view must stay
untouched."""
import numpy as np
import pytest

import synth
from gpu_util import assert_layer_close, dev

pytestmark = pytest.mark.gpu


def row_offsets(t):
    """byte offset of every row of a torch view, in ggml row order (row_offset of
    src/exl3-ggml.cpp:11-17): row r = i1 + ne1 (i2 + ne2 i3) with ne from the reversed shape"""
    es = t.element_size()
    ne = list(reversed(t.shape))[1:] + [1] * (4 - t.dim())
    nb = [s * es for s in reversed(t.stride())][1:] + [0] * (4 - t.dim())
    offs = []
    for r in range(ne[0] * ne[1] * ne[2]):
        i1, rest = r % ne[0], r // ne[0]
        i2, i3 = rest % ne[1], rest // ne[1]
        offs.append(i1 * nb[0] + i2 * nb[1] + i3 * nb[2])
    return offs


def gather_rows(base, view, row_len, np_dtype):
    """rows of a view of the flat torch buffer `base`, read from the buffer's bytes at row_offset"""
    raw = base.cpu().numpy().reshape(-1).view(np.uint8)
    start = view.data_ptr() - base.data_ptr()
    es = np.dtype(np_dtype).itemsize
    return np.stack([raw[start + o:start + o + row_len * es].view(np_dtype) for o in row_offsets(view)])


def make_layer(seed, k, n, bits):
    p = synth.packed_tiles(seed, k, n, bits)
    su, sv = synth.layer_scales(seed, k, n)
    return synth.pack_records(p, su, sv, bits).view(np.uint8)


CASES = {
    # x: rows 1..3 of a [2, 5, k] buffer (nb2 = 5 nb1, not 3 nb1); y dense [2, 3, n]
    "sliced_x": dict(xshape=(2, 5), xsel=lambda b: b[:, 1:4, :], yshape=(2, 3), ysel=lambda b: b),
    # x permuted: [3, 2, k] buffer viewed as [2, 3, k] (nb1 = 2 k es, nb2 = k es); y with a padded row stride
    "permuted_x_padded_y": dict(xshape=(3, 2), xsel=lambda b: b.permute(1, 0, 2), yshape=(2, 3),
                                ysel=lambda b: b[:, :, :-128], ypad=128),
    # both permuted: every row its own call
    "permuted_both": dict(xshape=(3, 2), xsel=lambda b: b.permute(1, 0, 2), yshape=(3, 2),
                          ysel=lambda b: b.permute(1, 0, 2)),
    # 4-D: ne = [k, 2, 2, 3] with a gap between the outer slices; 12 rows collapse into runs
    "four_d_gaps": dict(xshape=(3, 2, 3), xsel=lambda b: b[:, :, 1:3, :], yshape=(3, 2, 2), ysel=lambda b: b),
}


@pytest.mark.parametrize("case", list(CASES))
@pytest.mark.parametrize("xdt", ["f16", "f32"])
def test_mul_mat_nd_views(amd, oracle, case, xdt):
    import torch
    c = CASES[case]
    k, n, bits = 1024, 640, 4
    print(f"  mul_mat_nd {case} x={xdt} k={k} n={n}", flush=True)
    rec = make_layer(77, k, n, bits)
    tdt = torch.float16 if xdt == "f16" else torch.float32
    npdt = np.float16 if xdt == "f16" else np.float32
    g = torch.Generator().manual_seed(5)
    xbase = torch.randn(*c["xshape"], k, generator=g).to(tdt).cuda()
    xv = c["xsel"](xbase)
    pad = c.get("ypad", 0)
    ybase = torch.full((*c["yshape"], n + pad), 7.0, dtype=torch.float32).cuda()
    yv = c["ysel"](ybase)
    assert tuple(yv.shape[:-1]) == tuple(xv.shape[:-1]) and yv.shape[-1] == n
    amd.mul_mat_nd(dev(rec), bits, k, n, xv, yv)
    torch.cuda.synchronize()
    xrows = gather_rows(xbase, xv, k, npdt).astype(np.float32)
    want = oracle.mul_mat(rec, bits, 2, k, n, xrows)
    got = gather_rows(ybase, yv, n, np.float32)
    assert_layer_close(got, want, what=f"mul_mat_nd {case} {xdt}")
    # nothing outside the view was written
    mask = torch.ones_like(ybase, dtype=torch.bool)
    yv_mask = c["ysel"](mask)
    yv_mask.fill_(False)
    assert torch.all(ybase[mask] == 7.0)


def test_mul_mat_nd_matches_2d_call(amd):
    """a dense view through the N-D entry is one exl3_hip_mul_mat call: bit-identical"""
    import torch
    k, n, bits, rows = 2048, 768, 3, 5
    rec = dev(make_layer(12, k, n, bits))
    x = torch.randn(rows, k, generator=torch.Generator().manual_seed(3)).half().cuda()
    y2 = amd.mul_mat(rec, bits, k, n, x)
    ynd = torch.empty(rows, n, dtype=torch.float32, device="cuda")
    amd.mul_mat_nd(rec, bits, k, n, x, ynd)
    torch.cuda.synchronize()
    assert torch.equal(y2, ynd)


@pytest.mark.parametrize("odt", ["f32", "f16"])
def test_get_rows_nd_views(amd, oracle, odt):
    import torch
    k, n, bits = 512, 640, 6
    print(f"  get_rows_nd out={odt}", flush=True)
    rec_h = make_layer(31, k, n, bits)
    rec = dev(rec_h)
    # ids: every other column of a [2, 6] buffer -> ne = [3, 2], nb0 = 8, nb1 = 24
    idbuf = torch.tensor([[0, -5, n - 1, -5, 128, -5], [n // 2, -5, 1, -5, 333, -5]], dtype=torch.int32).cuda()
    ids = idbuf[:, ::2]
    tdt = torch.float32 if odt == "f32" else torch.float16
    npdt = np.float32 if odt == "f32" else np.float16
    obase = torch.full((2, 3, k + 64), 3.0, dtype=tdt).cuda()
    out = obase[:, :, 32:32 + k]
    amd.get_rows_nd(rec, bits, k, n, ids, out)
    torch.cuda.synchronize()
    flat_ids = ids.cpu().numpy().reshape(-1)
    want = oracle.get_rows(rec_h, bits, 2, k, n, flat_ids)
    got = gather_rows(obase, out, k, npdt)
    if odt == "f32":
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    else:
        assert np.array_equal(got.view(np.uint16), want.astype(np.float16).view(np.uint16))
    assert torch.all(obase[:, :, :32] == 3.0) and torch.all(obase[:, :, 32 + k:] == 3.0)


def test_mul_mat_nd_random_views(amd, oracle):
    """Seeded random 4-D views: x and y each a permutation of their three row
    dimensions, sliced from larger buffers (gaps between rows and slices), fp16 or
    fp32 x; every row checked against the oracle through row_offset, and nothing
    outside y's view written."""
    import itertools
    import torch
    k, n, bits = 512, 384, 3
    rec = make_layer(91, k, n, bits)
    rd = dev(rec)
    rng = np.random.default_rng(2026)
    perms = list(itertools.permutations(range(3)))
    for case in range(12):
        shape = tuple(int(v) for v in rng.integers(1, 4, size=3))   # row dimensions (outer .. inner)
        xdt = torch.float16 if case % 2 == 0 else torch.float32
        npdt = np.float16 if xdt == torch.float16 else np.float32
        g = torch.Generator().manual_seed(100 + case)
        px, py = perms[int(rng.integers(len(perms)))], perms[int(rng.integers(len(perms)))]
        pad_x = tuple(int(v) for v in rng.integers(0, 2, size=3))
        pad_y = tuple(int(v) for v in rng.integers(0, 2, size=3))
        # buffers laid out in the permuted order, one spare slice per padded dimension
        xs = tuple(shape[p] + pad_x[i] for i, p in enumerate(px))
        ys = tuple(shape[p] + pad_y[i] for i, p in enumerate(py))
        xbase = torch.randn(*xs, k + 32, generator=g).to(xdt).cuda()
        ybase = torch.full((*ys, n + 64), 7.0, dtype=torch.float32).cuda()
        inv_x, inv_y = np.argsort(px), np.argsort(py)
        xv = xbase[tuple(slice(0, shape[p]) for p in px) + (slice(16, 16 + k),)].permute(*inv_x, 3)
        yv = ybase[tuple(slice(0, shape[p]) for p in py) + (slice(0, n),)].permute(*inv_y, 3)
        assert tuple(xv.shape) == shape + (k,) and tuple(yv.shape) == shape + (n,)
        print(f"  random view {case}: rows {shape} x perm {px} y perm {py} x={xdt}", flush=True)
        amd.mul_mat_nd(rd, bits, k, n, xv, yv)
        torch.cuda.synchronize()
        want = oracle.mul_mat(rec, bits, 2, k, n, gather_rows(xbase, xv, k, npdt).astype(np.float32))
        assert_layer_close(gather_rows(ybase, yv, n, np.float32), want, what=f"random view {case}")
        mask = torch.ones_like(ybase, dtype=torch.bool)
        mask[tuple(slice(0, shape[p]) for p in py) + (slice(0, n),)] = False
        assert torch.all(ybase[mask] == 7.0), f"random view {case}: bytes outside the view written"
