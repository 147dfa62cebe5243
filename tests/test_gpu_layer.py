"""GPU layer parity: exl3_hip_mul_mat against the oracle's restatement of
ggml_exl3_mul_mat (src/exl3-ggml.cpp:51-92).  Tolerance: max-abs <= 1e-2 and
relative L2 <= 1e-3 on fp16 or fp32 outputs."""
from pathlib import Path

import numpy as np
import pytest

import synth
from gpu_util import assert_layer_close, dev, layer_stats

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"
THREADS = 8


def make_layer(seed, k, n, bits):
    p = synth.packed_tiles(seed, k, n, bits)
    su, sv = synth.layer_scales(seed, k, n)
    return synth.pack_records(p, su, sv, bits).view(np.uint8)


def run(amd, rec_d, bits, k, n, x, cb=2, out_dtype=None, **kw):
    import torch
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    y = amd.mul_mat(rec_d, bits, k, n, xd, codebook=cb, out_dtype=out_dtype or torch.float32, **kw)
    torch.cuda.synchronize()
    return y.float().cpu().numpy()


def test_golden_layer(amd):
    d = np.load(GOLD / "layer.npz", allow_pickle=False)
    k, n, bits, cb, rows = (int(v) for v in d["meta"])
    y = run(amd, dev(d["records"]), bits, k, n, d["x"], cb)
    ma, rl = layer_stats(y, d["y"])
    print(f"  golden layer vs float64: max_abs={ma:.2e} rel_l2={rl:.2e}", flush=True)
    assert rl < 1e-5
    assert np.sum((y - d["y_from_reconstruct"]) ** 2) / np.sum(d["y_from_reconstruct"] ** 2) < 1e-5


def test_c1_layer(amd, oracle):
    """k=2048 in, n=6144 out, 4 bits, batch 1, fp16 activations"""
    import torch
    k, n, bits = 2048, 6144, 4
    rec = make_layer(101, k, n, bits)
    x = synth.activations(102, 1, k)
    ref = oracle.mul_mat(rec, bits, 2, k, n, x, threads=THREADS)
    rd = dev(rec)
    assert_layer_close(run(amd, rd, bits, k, n, x), ref, what="C1 f32 out")
    assert_layer_close(run(amd, rd, bits, k, n, x, out_dtype=torch.float16), ref, what="C1 f16 out")


@pytest.mark.parametrize("bits", range(1, 9))
def test_all_rates_and_codebooks(amd, oracle, bits):
    k, n = 384, 384
    rec = make_layer(bits * 31, k, n, bits)
    rd = dev(rec)
    for cb in range(3):
        for rows in (1, 3, 8, 12, 24):
            x = synth.activations(bits * 100 + cb * 10 + rows, rows, k)
            ref = oracle.mul_mat(rec, bits, cb, k, n, x)
            assert_layer_close(run(amd, rd, bits, k, n, x, cb), ref, what=f"bits={bits} cb={cb} rows={rows}")


@pytest.mark.parametrize("rows", [1, 2, 4, 8, 9, 12, 14, 15, 16, 17, 24, 32])
def test_c3_full_size_gemv(amd, oracle, rows):
    """4096 x 14336 at 4 bits (k=14336 in, n=4096 out), ragged decode batches up to 32
    rows: the GEMV to 14 rows (rows 9..14 use its second block of MFMA columns), the
    GEMM's 32-row tiles above"""
    k, n, bits = 14336, 4096, 4
    rec = make_layer(303, k, n, bits)
    x = synth.activations(304 + rows, rows, k)
    ref = oracle.mul_mat(rec, bits, 2, k, n, x, threads=THREADS)
    y = run(amd, dev(rec), bits, k, n, x)
    ma, rl = assert_layer_close(y, ref, what=f"C3 rows={rows}")
    if rows <= 14:  # exl3_hip_mul_mat runs one matrix on the GEMV up to 14 rows (include/exl3_hip.h)
        assert rl < 1e-5  # hi/lo activation split keeps the GEMV at fp32-level accuracy


@pytest.mark.parametrize("k,n,bits", [(14336, 4096, 4), (6144, 2048, 3), (2048, 6144, 4)])
def test_gemv_rows_match_one_row_bitwise(amd, k, n, bits):
    """Every row of a 2..14-row GEMV call equals the one-row call of that row bit
    for bit (fp32 output): each row count prepares H128(x su) with the same
    roundings and the same fp16 hi/lo split, and each output column sums the same
    products in the same order.  A prep whose hi and lo came from two different
    roundings of one value (an fp16 conversion fused with the product for one use
    and not the other) shows here as single rows that differ."""
    rec = make_layer(430, k, n, bits)
    rd = dev(rec)
    x = synth.activations(431, 14, k)
    ones = np.concatenate([run(amd, rd, bits, k, n, x[r:r + 1]) for r in range(14)])
    for rows in (2, 4, 8, 9, 12, 14):
        y = run(amd, rd, bits, k, n, x[:rows])
        bad = [r for r in range(rows) if not np.array_equal(y[r], ones[r])]
        print(f"  k={k} n={n} rows={rows}: rows differing from one-row calls {bad}", flush=True)
        assert not bad


@pytest.mark.parametrize("k,n,bits", [(2048, 2048, 6), (2048, 512, 6), (6144, 2048, 3), (14336, 4096, 4)])
@pytest.mark.parametrize("rows", [15, 16])
def test_rows_15_16_short_k_on_gemv(amd, oracle, k, n, bits, rows):
    """One matrix at 15..16 rows runs the two-block hi/lo GEMV when a GEMV
    workgroup prepares at most 64 (record, row) blocks (short k: the q/k/v/o,
    gate/up and down projections of the 2B model), the GEMM's 32-row tiles
    otherwise (k = 14336).  The hi/lo split shows in the accuracy: rel-L2 < 1e-5
    on the GEMV against ~3e-4 with the GEMM's fp16 activations."""
    rec = make_layer(420 + k // 128 + rows, k, n, bits)
    x = synth.activations(421 + rows, rows, k)
    ref = oracle.mul_mat(rec, bits, 2, k, n, x, threads=THREADS)
    ma, rl = assert_layer_close(run(amd, dev(rec), bits, k, n, x), ref, what=f"k={k} n={n} rows={rows}")
    if k <= 8192:
        assert rl < 1e-5
    else:
        assert rl > 1e-5  # the GEMM: fp16 activations


@pytest.mark.parametrize("rows", [33, 37, 128, 300])
def test_gemm_rows(amd, oracle, rows):
    k, n, bits = 1024, 384, 4
    rec = make_layer(400 + rows, k, n, bits)
    x = synth.activations(401 + rows, rows, k)
    ref = oracle.mul_mat(rec, bits, 2, k, n, x, threads=THREADS)
    assert_layer_close(run(amd, dev(rec), bits, k, n, x), ref, what=f"GEMM rows={rows}")


@pytest.mark.parametrize("k,n,rows", [(1024, 384, 64), (2048, 640, 48), (512, 384, 40), (1024, 384, 17),
                                      (2048, 640, 32), (512, 384, 24), (128, 384, 40), (128, 384, 24)])
def test_gemm_short_row_tiles(amd, oracle, k, n, rows):
    """Rows 17..32 run 32-row tiles (4 column quarters), rows 33..64 64-row tiles
    (2 row waves x 4 column quarters); both always split k (at k = 512 into four
    splits of one record each), and at k = 128 (one record) no split is
    possible, so the call runs the 128-row tile without one."""
    bits = 3
    rec = make_layer(410 + rows, k, n, bits)
    x = synth.activations(411 + rows, rows, k)
    ref = oracle.mul_mat(rec, bits, 2, k, n, x, threads=THREADS)
    assert_layer_close(run(amd, dev(rec), bits, k, n, x), ref, what=f"GEMM k={k} n={n} rows={rows}")


@pytest.mark.parametrize("rows", [100, 200, 300])
def test_gemm_unsplit_tiles(amd, oracle, rows):
    """At k = 256, n = 4096 the 128-, 256- and 512-row tiles run without a k split
    (32 column groups: the split partials would cost more than the second
    record's decode saves), so each workgroup sums both records and applies H128
    and sv itself."""
    k, n, bits = 256, 4096, 4
    rec = make_layer(420 + rows, k, n, bits)
    x = synth.activations(421 + rows, rows, k)
    ref = oracle.mul_mat(rec, bits, 2, k, n, x, threads=THREADS)
    assert_layer_close(run(amd, dev(rec), bits, k, n, x), ref, what=f"GEMM k={k} n={n} rows={rows}")


def test_k4096_n14336_gemv_and_gemm(amd, oracle):
    """The 4096 x 14336 weight in the gate/up orientation (k=4096 in, n=14336 out):
    the GEMV at rows 1 and 8 (112 column groups x 4 k-splits, hi/lo activations,
    fp32-level accuracy) and the M=512 GEMM (512-row tiles, 2 k-splits) on
    sampled rows, against the oracle."""
    k, n, bits = 4096, 14336, 4
    rec = make_layer(440, k, n, bits)
    rd = dev(rec)
    for rows in (1, 8):
        x = synth.activations(441 + rows, rows, k)
        ref = oracle.mul_mat(rec, bits, 2, k, n, x, threads=THREADS)
        _, rl = assert_layer_close(run(amd, rd, bits, k, n, x), ref, what=f"k=4096 n=14336 rows={rows}")
        assert rl < 1e-5
    x = synth.activations(450, 512, k)
    y = run(amd, rd, bits, k, n, x)
    pick = np.array([0, 1, 255, 256, 511])
    ref = oracle.mul_mat(rec, bits, 2, k, n, x[pick], threads=THREADS)
    assert_layer_close(y[pick], ref, what="k=4096 n=14336 M=512 sampled rows")


def test_c5_prefill_sampled(amd, oracle):
    """M=512 rows against 4096 x 14336 at 4 bits; 8 sampled rows against the oracle,
    all rows against the GEMV path on the same inputs."""
    import torch
    k, n, bits, rows = 14336, 4096, 4, 512
    rec = make_layer(505, k, n, bits)
    x = synth.activations(506, rows, k)
    rd = dev(rec)
    y = run(amd, rd, bits, k, n, x, out_dtype=torch.float16)
    pick = np.array([0, 1, 127, 128, 255, 300, 510, 511])
    ref = oracle.mul_mat(rec, bits, 2, k, n, x[pick], threads=THREADS)
    assert_layer_close(y[pick], ref, what="C5 sampled rows")
    for r0 in (0, 504):
        yg = run(amd, rd, bits, k, n, x[r0:r0 + 8])
        assert_layer_close(y[r0:r0 + 8], yg, what=f"C5 GEMM vs GEMV rows {r0}..")


def test_f32_input_and_strides(amd, oracle):
    import torch
    k, n, bits = 512, 256, 3
    rec = make_layer(600, k, n, bits)
    rd = dev(rec)
    for rows in (5, 11, 20, 40):
        x16 = synth.activations(601, rows, k)
        ref = oracle.mul_mat(rec, bits, 2, k, n, x16)
        xpad = np.zeros((rows, k + 64), np.float32)
        xpad[:, :k] = x16.astype(np.float32)
        xd = torch.from_numpy(xpad).cuda()[:, :k]
        ybig = torch.full((rows, n + 32), 7.0, dtype=torch.float32, device="cuda")
        amd.mul_mat(rd, bits, k, n, xd, y=ybig[:, :n])
        torch.cuda.synchronize()
        yb = ybig.cpu().numpy()
        assert np.all(yb[:, n:] == 7.0)
        assert_layer_close(yb[:, :n], ref, what=f"f32 strided rows={rows}")


def test_deterministic_and_workspaces(amd):
    import torch
    k, n, bits = 4096, 1024, 4
    rec = dev(make_layer(700, k, n, bits))
    for rows in (1, 8, 13, 64):
        x = torch.from_numpy(synth.activations(701, rows, k)).cuda()
        y1 = amd.mul_mat(rec, bits, k, n, x).clone()
        y2 = amd.mul_mat(rec, bits, k, n, x).clone()
        ws = amd.new_workspace(k, n, rows)
        y3 = amd.mul_mat(rec, bits, k, n, x, workspace=ws).clone()
        y4 = amd.mul_mat(rec, bits, k, n, x, workspace=ws).clone()
        torch.cuda.synchronize()
        assert torch.equal(y1, y2) and torch.equal(y1, y3) and torch.equal(y1, y4), rows
        small = torch.zeros(256, dtype=torch.uint8, device="cuda")
        with pytest.raises(amd.Exl3Error) as e:
            amd.mul_mat(rec, bits, k, n, x, workspace=small)
        assert e.value.status == amd.WORKSPACE_TOO_SMALL


def test_invalid_parameters_rejected(amd):
    import torch
    rec = torch.zeros(2048 * 4 + 512, dtype=torch.uint8, device="cuda")
    x = torch.zeros((1, 128), dtype=torch.float16, device="cuda")
    for bits, cb, k, n in [(0, 2, 128, 128), (9, 2, 128, 128), (4, 3, 128, 128), (4, 2, 64, 128), (4, 2, 128, 200)]:
        with pytest.raises(amd.Exl3Error) as e:
            amd.mul_mat(rec, bits, k, n, x if k == 128 else torch.zeros((1, k), dtype=torch.float16, device="cuda"),
                        codebook=cb)
        assert e.value.status == amd.INVAL_PARAMS


def test_c4_projection_set(amd, oracle):
    """decoder-layer projections at batch 8, mixed 3/4/6 bits, x ~ N(0, 0.5)"""
    shapes = [("q", 2048, 2048, 6), ("k", 2048, 512, 6), ("v", 2048, 512, 6), ("o", 2048, 2048, 6),
              ("gate", 2048, 6144, 4), ("up", 2048, 6144, 4), ("down", 6144, 2048, 3)]
    for i, (name, k, n, bits) in enumerate(shapes):
        rec = make_layer(800 + i, k, n, bits)
        x = synth.activations(810 + i, 8, k, sigma=0.5)
        ref = oracle.mul_mat(rec, bits, 2, k, n, x, threads=THREADS)
        assert_layer_close(run(amd, dev(rec), bits, k, n, x), ref, what=f"C4 {name}")


def test_linearity_full_size(amd):
    import torch
    k, n, bits = 14336, 4096, 4
    rec = dev(make_layer(900, k, n, bits))
    for rows in (4, 64):
        x1 = synth.activations(901, rows, k).astype(np.float32)
        x2 = synth.activations(902, rows, k).astype(np.float32)
        ys = [run(amd, rec, bits, k, n, v) for v in (x1, x2, x1 + x2)]
        assert_layer_close(ys[2], ys[0] + ys[1], what=f"linearity rows={rows}")


@pytest.mark.parametrize("rows", [1, 5, 14, 24, 37])
def test_graph_replay_matches_eager(amd, oracle, rows):
    """A HIP graph of mul_mat calls (split-K counters self-reset, no memset
    nodes) replays bit-identically, with eager work between the replays."""
    import torch
    k, n, bits = 4096, 1024, 4
    recs = [make_layer(700 + i, k, n, bits) for i in range(2)]
    rds = [dev(r) for r in recs]
    x = torch.from_numpy(synth.activations(710 + rows, rows, k)).cuda()
    ws = amd.new_workspace(k, n, rows)
    ys = [torch.empty((rows, n), dtype=torch.float32, device="cuda") for _ in range(2)]
    eager = []
    for i in range(2):
        amd.mul_mat(rds[i], bits, k, n, x, y=ys[i], workspace=ws)
        eager.append(ys[i].clone())
    torch.cuda.synchronize()
    for i in range(2):
        ref = oracle.mul_mat(recs[i], bits, 2, k, n, x.cpu().numpy(), threads=THREADS)
        assert_layer_close(eager[i].cpu().numpy(), ref, what=f"eager rows={rows} layer {i}")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(2):
            amd.mul_mat(rds[i], bits, k, n, x, y=ys[i], workspace=ws)
    for rep in range(4):
        for y in ys:
            y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for i in range(2):
            assert torch.equal(ys[i], eager[i]), f"replay {rep} layer {i} rows={rows}"
        # eager call on the same workspace between replays
        amd.mul_mat(rds[1], bits, k, n, x, y=ys[1], workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(ys[1], eager[1])


def test_one_workspace_serves_mixed_row_counts(amd):
    """Calls of different row counts (GEMV and GEMM, several m-tiles) share a
    caller workspace sized for the largest, and the internal workspace, in any
    order: every result equals the one from a fresh workspace."""
    import torch
    k, n, bits = 2048, 4096, 4
    rd = dev(make_layer(820, k, n, bits))
    seq = [300, 100, 300, 5, 300, 1, 37, 300, 8, 129, 16, 11, 300, 9, 32, 20, 300, 17]
    xs = {r: torch.from_numpy(synth.activations(821 + r, r, k)).cuda() for r in set(seq)}
    fresh = {}
    for r in set(seq):
        ws = amd.new_workspace(k, n, r)
        fresh[r] = amd.mul_mat(rd, bits, k, n, xs[r], workspace=ws).clone()
    torch.cuda.synchronize()
    shared = amd.new_workspace(k, n, max(seq))
    for i, r in enumerate(seq):
        y_shared = amd.mul_mat(rd, bits, k, n, xs[r], workspace=shared)
        y_internal = amd.mul_mat(rd, bits, k, n, xs[r])
        torch.cuda.synchronize()
        assert torch.equal(y_shared, fresh[r]), f"caller workspace, call {i} rows={r}"
        assert torch.equal(y_internal, fresh[r]), f"internal workspace, call {i} rows={r}"


@pytest.mark.parametrize("rows", [1, 3, 8, 12, 16, 20, 32, 40])
def test_group_matches_single_layers(amd, oracle, rows):
    """q/k/v and gate/up of one decoder layer through exl3_hip_mul_mat_group: one GEMV
    launch (rows <= 32; above 16 after one activation pass for all matrices) that serves
    several matrices sharing x; each output within the layer tolerance of the oracle,
    and above (one call per matrix) equal to mul_mat"""
    import torch
    for k, shapes, bits in [(2048, [2048, 512, 512], 6), (2048, [6144, 6144], 4)]:
        recs = [make_layer(700 + i + bits, k, n, bits) for i, n in enumerate(shapes)]
        x = synth.activations(800 + rows, rows, k)
        xd = torch.from_numpy(x).cuda()
        ys = amd.mul_mat_group([(dev(r), n) for r, n in zip(recs, shapes)], bits, k, xd)
        for i, (r, n) in enumerate(zip(recs, shapes)):
            y = ys[i].cpu().numpy()
            assert_layer_close(y, oracle.mul_mat(r, bits, 2, k, n, x), what=f"group {i} n={n} rows={rows}")
            if rows > amd.lib().exl3_hip_gemv_max_rows():
                single = amd.mul_mat(dev(r), bits, k, n, xd).cpu().numpy()
                assert np.array_equal(y, single)
    L = amd.lib()
    assert L.exl3_hip_mul_mat_group(None, 1, 4, 2, 2048, None, 1, 1, 2048, 1, None, 0, None) == 1


@pytest.mark.parametrize("rows", [520, 33])
def test_group_workspace_of_documented_size(amd, rows):
    """gate/up (k = 2048, n = 8192 each) at rows where the group runs one exl3_hip_mul_mat
    per matrix, whose split partials need more than the total width's plan: a caller
    workspace of exactly exl3_hip_mul_mat_group_workspace_bytes is accepted, and each
    output equals exl3_hip_mul_mat's bit for bit"""
    import torch
    k, n, bits = 2048, 8192, 4
    print(f"  group workspace rows={rows}", flush=True)
    recs = [dev(make_layer(760 + i, k, n, bits)) for i in range(2)]
    x = torch.from_numpy(synth.activations(761, rows, k)).cuda()
    nbytes = amd.group_workspace_bytes(k, [n, n], rows)
    assert nbytes >= amd.lib().exl3_hip_mul_mat_workspace_bytes(k, n, rows)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    amd.workspace_init(ws)
    ys = amd.mul_mat_group([(r, n) for r in recs], bits, k, x, workspace=ws)
    for r, y in zip(recs, ys):
        assert torch.equal(y, amd.mul_mat(r, bits, k, n, x))


def test_concurrent_streams(amd):
    """Calls interleaved on two streams (default priority) at once: with internal
    workspaces (one per device and stream) and with a caller workspace per stream,
    every result equals the same call made alone (the layer is deterministic)."""
    import torch
    k, n, bits = 4096, 2048, 4
    recs = [dev(make_layer(900 + i, k, n, bits)) for i in range(2)]
    row_counts = (1, 8, 13, 40)
    xs = [torch.from_numpy(synth.activations(910 + r, r, k)).cuda() for r in row_counts]
    ref = [[amd.mul_mat(recs[i], bits, k, n, x).clone() for x in xs] for i in range(2)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    wss = [amd.new_workspace(k, n, max(row_counts)) for _ in range(2)]
    torch.cuda.synchronize()
    for use_ws in (False, True):
        for rep in range(3):
            outs = [[None] * len(xs) for _ in range(2)]
            for j, x in enumerate(xs):
                for i in range(2):
                    with torch.cuda.stream(streams[i]):
                        outs[i][j] = amd.mul_mat(recs[i], bits, k, n, x, stream=streams[i],
                                                 workspace=wss[i] if use_ws else None)
            torch.cuda.synchronize()
            for i in range(2):
                for j, r in enumerate(row_counts):
                    assert torch.equal(outs[i][j], ref[i][j]), f"stream {i} rows={r} rep={rep} ws={use_ws}"


def test_one_workspace_serves_mixed_widths(amd):
    """One caller workspace shared by layers of different n and both kernels: a
    GEMM call at n=2048 (its activation staging sits behind the split-K
    exchange), then GEMV calls at n=14336 (more column groups) and a gate/up
    group (n = 2 x 6144).  The exchange does not depend on n, so no call writes
    over another's: every result equals the one from a fresh workspace, over two
    rounds of the sequence."""
    import torch
    cases = {  # name: (k, [n...], rows, bits)
        "gemm_n2048": (4096, [2048], 64, 4),
        "gemv_n14336": (4096, [14336], 1, 4),
        "gemv_n14336_r8": (4096, [14336], 8, 4),
        "group_gate_up": (4096, [6144, 6144], 3, 4),
        "gemv_n2048_r24": (4096, [2048], 24, 4),
    }
    recs = {name: [dev(make_layer(950 + 7 * i + j, k, n, bits)) for j, n in enumerate(ns)]
            for i, (name, (k, ns, rows, bits)) in enumerate(cases.items())}
    xs = {name: torch.from_numpy(synth.activations(970 + i, rows, k)).cuda()
          for i, (name, (k, ns, rows, bits)) in enumerate(cases.items())}

    def call(name, ws):
        k, ns, rows, bits = cases[name]
        if len(ns) > 1:
            return [y.clone() for y in amd.mul_mat_group([(r, n) for r, n in zip(recs[name], ns)], bits, k, xs[name],
                                                         workspace=ws)]
        return [amd.mul_mat(recs[name][0], bits, k, ns[0], xs[name], workspace=ws).clone()]

    fresh = {}
    for name, (k, ns, rows, bits) in cases.items():
        fresh[name] = call(name, amd.new_workspace(k, sum(ns), rows))
    torch.cuda.synchronize()
    size = max(amd.workspace_bytes(k, sum(ns), rows) for k, ns, rows, _ in cases.values())
    shared = torch.zeros(size, dtype=torch.uint8, device="cuda")
    for rnd in range(2):
        for name in ("gemm_n2048", "gemv_n14336", "group_gate_up", "gemm_n2048", "gemv_n14336_r8",
                     "gemv_n2048_r24", "gemv_n14336", "group_gate_up"):
            got = call(name, shared)
            torch.cuda.synchronize()
            for a, b in zip(got, fresh[name]):
                assert torch.equal(a, b), f"round {rnd}: {name} differs from a fresh workspace"


@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")  # the refused capture records nothing
def test_internal_workspace_under_capture(amd):
    """With no caller workspace, a call captured into a HIP graph before any
    uncaptured call of its size is refused with EXL3_WORKSPACE_TOO_SMALL (the
    internal workspace cannot grow during capture) instead of allocating; after
    one uncaptured call the same capture succeeds and replays equal eager calls."""
    import torch
    k, n, bits, rows = 1024, 640, 4, 2   # a shape no other test uses: its internal workspace is new
    rd = dev(make_layer(990, k, n, bits))
    x = torch.from_numpy(synth.activations(991, rows, k)).cuda()
    y = torch.empty((rows, n), dtype=torch.float16, device="cuda")
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with pytest.raises(amd.Exl3Error) as err:
        with torch.cuda.graph(g, stream=s):
            amd.mul_mat(rd, bits, k, n, x, y=y, stream=s)
    assert err.value.status == amd.WORKSPACE_TOO_SMALL
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        eager = amd.mul_mat(rd, bits, k, n, x, out_dtype=torch.float16, stream=s).clone()  # grows the workspace
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        amd.mul_mat(rd, bits, k, n, x, y=y, stream=s)
    for _ in range(3):
        y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager)


# bytes every workspace starts with: the 16 MiB of split-K hand-off words (zero
# between calls)
SHARED_PREFIX = 16 << 20


def test_exchange_left_empty(amd):
    """The split-K hand-off leaves the workspace's exchange zero after every GEMV
    call (the workgroups that sum the splits empty what they read), and GEMM
    calls never write there: a caller workspace used for GEMV calls of 1..32
    rows, a group call and GEMM calls is zero over its first SHARED_PREFIX bytes
    after each call, and every result equals the one from a fresh workspace."""
    import torch
    k, n, bits = 14336, 4096, 4
    rd = dev(make_layer(303, k, n, bits))
    seq = [1, 8, 16, 32, 64, 2, 17, 512, 9, 1]
    ws = amd.new_workspace(k, n, max(seq))
    assert ws.numel() >= SHARED_PREFIX
    for i, rows in enumerate(seq):
        x = torch.from_numpy(synth.activations(1300 + rows, rows, k)).cuda()
        y = amd.mul_mat(rd, bits, k, n, x, workspace=ws).clone()
        fresh = amd.mul_mat(rd, bits, k, n, x, workspace=amd.new_workspace(k, n, rows))
        torch.cuda.synchronize()
        assert torch.equal(y, fresh), f"call {i} rows={rows}"
        nz = int(torch.count_nonzero(ws[:SHARED_PREFIX]))
        assert nz == 0, f"call {i} rows={rows}: {nz} nonzero bytes left in the exchange"
    mats = [(dev(make_layer(1400 + j, 2048, 6144, 4)), 6144) for j in range(2)]
    wsg = amd.new_workspace(2048, 2 * 6144, 8)
    for rows in (3, 8):
        x = torch.from_numpy(synth.activations(1410 + rows, rows, 2048)).cuda()
        amd.mul_mat_group(mats, 4, 2048, x, workspace=wsg)
        torch.cuda.synchronize()
        assert int(torch.count_nonzero(wsg[:SHARED_PREFIX])) == 0, f"group rows={rows}"


def test_gemv_partials_beyond_exchange_run_as_gemm(amd):
    """k=16384, n=8320 at 32 rows: the GEMV's split partials (1040 column-group
    splits x 32 rows x 512 B = 17 MB) would not fit the 16 MiB exchange, so the
    call runs as a GEMM; at 16 rows they fit and the GEMV runs.  The 32-row
    result matches the two 16-row GEMV halves within the layer tolerance, and the
    workspace's exchange stays zero."""
    import torch
    k, n, bits = 16384, 8320, 2
    rd = dev(make_layer(1500, k, n, bits))
    x = torch.from_numpy(synth.activations(1501, 32, k)).cuda()
    ws = amd.new_workspace(k, n, 32)
    y32 = amd.mul_mat(rd, bits, k, n, x, workspace=ws)
    halves = torch.cat([amd.mul_mat(rd, bits, k, n, x[:16].contiguous(), workspace=ws),
                        amd.mul_mat(rd, bits, k, n, x[16:].contiguous(), workspace=ws)])
    torch.cuda.synchronize()
    assert_layer_close(y32.cpu().numpy(), halves.cpu().numpy().astype(np.float64), what="GEMM fallback vs GEMV")
    assert int(torch.count_nonzero(ws[:SHARED_PREFIX])) == 0


@pytest.mark.parametrize("rows", [1, 12, 20, 40])
def test_fp32_input_range(amd, oracle, rows):
    """fp32 activations up to the documented range (|x su| <= 5790 keeps the fp16
    xh = H128(x su)/sqrt(128) finite): sigma 1000 (|x| up to ~5000) matches the
    oracle within the layer tolerance, scaled to the output size, on the GEMV's hi/lo
    path (rows 1, 12), its fp16 path (20) and the GEMM (40).  Far beyond the range
    (sigma 1e6) the affected rows are not finite, as documented."""
    import torch
    k, n, bits = 1024, 384, 4
    rec = make_layer(1600, k, n, bits)
    rd = dev(rec)
    rng = np.random.default_rng(1601 + rows)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    big = x * np.float32(1000.0)
    big = np.clip(big, -5790.0, 5790.0).astype(np.float32)
    y = run(amd, rd, bits, k, n, big)
    ref = oracle.mul_mat(rec, bits, 2, k, n, big)
    scale = float(np.max(np.abs(ref)))
    ma, rl = layer_stats(y, ref)
    print(f"  fp32 range rows={rows}: max_abs={ma:.3e} (output scale {scale:.1f}) rel_l2={rl:.3e}", flush=True)
    assert np.all(np.isfinite(y))
    assert rl <= 1e-3 and ma <= 1e-2 * max(1.0, scale / 10.0)
    huge = (x * np.float32(1e6)).astype(np.float32)
    yh = run(amd, rd, bits, k, n, huge)
    assert not np.all(np.isfinite(yh))


@pytest.mark.parametrize("bits", range(1, 9))
def test_every_tile_class_rate_and_codebook(amd, oracle, bits):
    """Every kernel instance the layer dispatches to, for each rate and codebook:
    the GEMM's 32-, 64-, 128-, 256- and 512-row tiles (rows 24, 40, 100, 200, 300)
    and the grouped GEMV's 17..32-row mode with its separate activation prep
    (two matrices, rows 20), against the oracle at the layer tolerance."""
    import torch
    k, n = 512, 256
    rec = make_layer(1500 + bits, k, n, bits)
    rec2 = make_layer(1600 + bits, k, n, bits)
    rd, rd2 = dev(rec), dev(rec2)
    for cb in range(3):
        for rows in (24, 40, 100, 200, 300):
            x = synth.activations(1700 + 10 * bits + cb + rows, rows, k)
            ref = oracle.mul_mat(rec, bits, cb, k, n, x, threads=THREADS)
            assert_layer_close(run(amd, rd, bits, k, n, x, cb), ref, what=f"bits={bits} cb={cb} rows={rows}")
        x = synth.activations(1800 + 10 * bits + cb, 20, k)
        ys = amd.mul_mat_group([(rd, n), (rd2, n)], bits, k, torch.from_numpy(x).cuda(), codebook=cb)
        torch.cuda.synchronize()
        for r, y, tag in ((rec, ys[0], "a"), (rec2, ys[1], "b")):
            ref = oracle.mul_mat(r, bits, cb, k, n, x, threads=THREADS)
            assert_layer_close(y.cpu().numpy(), ref, what=f"group {tag} bits={bits} cb={cb} rows=20")
