"""GPU decode parity: every decoded fp16 weight bit-exact with the oracle and
with the golden vectors of the compiled reference codec."""
import hashlib
import json
import subprocess
from pathlib import Path

import numpy as np
import pytest

import synth
from gpu_util import dev, host_u16
from test_oracle import golden_matrix_inputs, read_exl3ref

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def test_codebook_all_states(amd, oracle):
    import torch
    states = torch.arange(65536, dtype=torch.int32).to(torch.int16).cuda()
    g = json.loads((GOLD / "codebook.json").read_text())
    for cb in range(3):
        print(f"  codebook cb={cb}", flush=True)
        out = host_u16(amd.codebook_values(states, cb))
        assert np.array_equal(out, oracle.codebook_table(cb)), cb
        assert sha(out.astype("<u2")) == g[str(cb)]["sha256"]


def test_decode_golden_tiles(amd):
    d = np.load(GOLD / "tiles.npz", allow_pickle=False)
    nt = d["packed"].shape[2]
    for bits in range(1, 9):
        for cb in range(3):
            print(f"  tiles bits={bits} cb={cb}", flush=True)
            up = d["packed"][bits - 1, cb, :, : 16 * bits].reshape(1, nt, 16 * bits)
            out = host_u16(amd.decode(dev(up), bits, 16, 16 * nt, codebook=cb))
            for t in range(nt):
                assert np.array_equal(out[:, 16 * t: 16 * t + 16].reshape(-1), d["decoded"][bits - 1, cb, t]), (bits, cb, t)


@pytest.mark.parametrize("bits", range(1, 9))
def test_decode_and_reconstruct_golden_matrices(amd, bits):
    mats = [m for m in json.loads((GOLD / "matrices.json").read_text()) if m["bits"] == bits]
    for m in mats:
        p, su, sv = golden_matrix_inputs(m)
        k, n, cb = m["k"], m["n"], m["cb"]
        print(f"  matrix bits={bits} cb={cb} {k}x{n}", flush=True)
        dp, dsu, dsv = dev(p), dev(su.view(np.uint16)), dev(sv.view(np.uint16))
        inner = host_u16(amd.decode(dp, bits, k, n, codebook=cb))
        assert sha(inner.astype("<u2")) == m["inner_sha256"]
        sl = host_u16(amd.decode(dp, bits, k, n, codebook=cb, first=32, count=48))
        assert np.array_equal(sl, inner[:, 32:80])
        orig = host_u16(amd.reconstruct(dp, bits, k, n, su=dsu, sv=dsv, codebook=cb))
        assert sha(orig.astype("<u2")) == m["original_sha256"]
        # the same weights through the record layout (packed on the GPU)
        rec = amd.pack_records(dp, dsu, dsv, bits, k, n)
        assert np.array_equal(rec.cpu().numpy(), synth.pack_records(p, su, sv, bits).view(np.uint8))
        assert np.array_equal(host_u16(amd.decode(rec, bits, k, n, codebook=cb, layout=amd.LAYOUT_RECORDS)), inner)
        assert np.array_equal(host_u16(amd.reconstruct(rec, bits, k, n, codebook=cb, layout=amd.LAYOUT_RECORDS)), orig)
        o2 = host_u16(amd.reconstruct(rec, bits, k, n, codebook=cb, layout=amd.LAYOUT_RECORDS, first=128, count=256))
        assert np.array_equal(o2, orig[:, 128:384])


def test_hadamard_bit_exact(amd):
    for case in json.loads((GOLD / "hadamard.json").read_text()):
        x = np.array(case["input"], dtype=np.uint32).view(np.float32)
        t = dev(x)
        amd.hadamard128(t)
        assert np.array_equal(t.cpu().numpy().view(np.uint32), np.array(case["output"], dtype=np.uint32))


@pytest.mark.parametrize("name", ["k4-cb2-128x256.exl3ref", "k3-cb0-128x128.exl3ref"])
def test_exl3ref_fixtures(amd, name):
    k, n, bits, cb, packed, su, sv, inner, orig = read_exl3ref(GOLD / name)
    dp = dev(packed)
    assert np.array_equal(host_u16(amd.decode(dp, bits, k, n, codebook=cb)), inner)
    got = host_u16(amd.reconstruct(dp, bits, k, n, su=dev(su), sv=dev(sv), codebook=cb))
    assert np.array_equal(got, orig)


def test_validate_records(amd):
    k, n, bits = 256, 256, 4
    p = synth.packed_tiles(12, k, n, bits)
    su, sv = synth.layer_scales(12, k, n)
    rec = synth.pack_records(p, su, sv, bits).view(np.uint8).copy()
    assert amd.validate_records(dev(rec), bits) == 1
    bad = rec.view(np.uint16).copy()
    bad[(3 * synth.group_bytes(bits) + 2048 * bits + 6) // 2] = 0xFC00  # -inf su in record 3
    assert amd.validate_records(dev(bad.view(np.uint8)), bits) == 0
    with pytest.raises(amd.Exl3Error):
        amd.validate_records(dev(rec[:-512]), bits)


@pytest.mark.parametrize("k,n,bits", [(2048, 6144, 4), (14336, 4096, 4), (2048, 151936 // 8 // 128 * 128, 6)])
def test_decode_full_size_records(amd, oracle, k, n, bits):
    print(f"  decode records {k}x{n} bits={bits}", flush=True)
    p = synth.packed_tiles(k + n + bits, k, n, bits)
    su, sv = synth.layer_scales(1, k, n)
    rec = synth.pack_records(p, su, sv, bits)
    out = host_u16(amd.decode(dev(rec.view(np.uint8)), bits, k, n, codebook=2, layout=amd.LAYOUT_RECORDS))
    assert np.array_equal(out, oracle.decode_records(rec, k, n, bits, 2))


@pytest.mark.parametrize("bits", [2, 3, 5, 6])
def test_decode_mixed_rates(amd, oracle, bits):
    k, n = 2048, 512
    p = synth.packed_tiles(bits * 7, k, n, bits)
    out = host_u16(amd.decode(dev(p), bits, k, n, codebook=2))
    assert np.array_equal(out, oracle.decode_inner(p, k, n, bits, 2))


def test_cpp_codec_api_program():
    """tests/cpp/test_codec_api.cpp: the C++ API (include/exl3_codec.h) driven
    like the reference's tests/test_codec.cpp, as a separate program built by
    build() against the in-tree library."""
    exe = Path(__file__).resolve().parent / "cpp" / "test_codec_api"
    assert exe.exists(), "tests/cpp/test_codec_api is built by __graft_entry__.build()"
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0 and "PASS" in r.stdout


REF_TEST_ON_HIP = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "test_codec_hip"


@pytest.mark.skipif(not REF_TEST_ON_HIP.exists(), reason="built only where the reference checkout was present")
def test_reference_codec_test_on_hip_library():
    """The reference's own codec test (tests/test_codec.cpp), compiled against
    this repository's include/ (exl3_codec.h, exl3-block.h) and linked with
    libexl3_hip.so by oracle/Makefile: its mul1 closed form, fp16 rounding,
    H128 involution, zero ring, rejections and VTCM planner checks all pass
    against the GPU-backed codec."""
    r = subprocess.run([str(REF_TEST_ON_HIP)], capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0 and r.stdout.startswith("PASS"), r.stdout + r.stderr


def test_decode_batch_matches_single_decodes(amd, oracle):
    """exl3_hip_decode_batch: 45 matrices of every rate (more than one launch's
    32 for 4 bits), upstream tiles, each bit-identical with its own
    exl3_hip_decode call; the small ones also with the oracle."""
    import torch
    g = torch.Generator(device="cuda")
    shapes = [(16, 16), (32, 48), (128, 128), (256, 512), (2048, 128), (128, 2064), (640, 784)]
    items, meta = [], []
    for j in range(45):
        bits = 4 if j >= 13 else 1 + j % 8
        k, n = shapes[j % len(shapes)]
        g.manual_seed(500 + j)
        p = torch.randint(-32768, 32768, (k * n * bits // 16,), generator=g, device="cuda",
                          dtype=torch.int32).to(torch.int16)
        items.append((p, bits, k, n, None))
        meta.append((p, bits, k, n))
    outs = amd.decode_batch(items, codebook=2)
    torch.cuda.synchronize()
    for (p, bits, k, n), out in zip(meta, outs):
        single = amd.decode(p, bits, k, n, codebook=2)
        torch.cuda.synchronize()
        assert torch.equal(out, single), (bits, k, n)
        if k * n <= 128 * 128:
            want = oracle.decode_inner(p.cpu().numpy().view(np.uint16), k, n, bits, 2)
            assert np.array_equal(host_u16(out), want), (bits, k, n)
    assert amd.decode_batch([], codebook=2) == []


def test_decode_batch_records_layout(amd):
    import torch
    items = []
    for j, (k, n, bits) in enumerate([(128, 256, 3), (256, 128, 6), (384, 384, 3), (128, 128, 2)]):
        rec = synth.pack_records(synth.packed_tiles(610 + j, k, n, bits), *synth.layer_scales(610 + j, k, n), bits)
        items.append((dev(rec.view(np.uint8)), bits, k, n, None))
    outs = amd.decode_batch(items, codebook=1, layout=amd.LAYOUT_RECORDS)
    for (rd, bits, k, n, _), out in zip(items, outs):
        single = amd.decode(rd, bits, k, n, codebook=1, layout=amd.LAYOUT_RECORDS)
        torch.cuda.synchronize()
        assert torch.equal(out, single), (bits, k, n)
