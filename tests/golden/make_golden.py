"""Generate the committed golden fixtures from the reference codec compiled
from its own sources (oracle/_ref/libexl3ref.so, built by `make -C oracle ref`).

Run in the build container only (the reference checkout does not travel):
    python tests/golden/make_golden.py
Outputs (all data, no code):
    codebook.json   sha256 of the full 65536-entry table per codebook + spot values
    tiles.npz       edge and random tiles for bits 1..8 x codebooks 0..2 and their decodes
    matrices.json   256x384 decode_inner / reconstruct digests per bits x codebook
    hadamard.json   H128 of fixed vectors (binary32 bit patterns)
    layer.npz       a small EXL3 layer: records, x, y (float64 expectation)
    *.exl3ref       two fixtures in the reference's EXL3REF1 format
                    (tools/exl3_verify.cpp:10, tests/generate_cuda_fixtures.py:82-85)
    get_rows.npz    GET_ROWS expectations computed the way ggml_exl3_get_rows
                    does (src/exl3-ggml.cpp:29-43): the reference exl3::reconstruct
                    of each 128x128 record, column id % 128, widened to fp32
Sections can be named to regenerate only those: make_golden.py get_rows
"""
import hashlib
import json
import struct
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
import synth  # noqa: E402
from oracle_lib import Reference  # noqa: E402


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def edge_tiles(bits, seed):
    w = 16 * bits
    tiles = np.zeros((6, 128), dtype=np.uint16)
    tiles[1, :w] = 0xFFFF
    tiles[2, :w] = 0xAAAA
    tiles[3, :w] = np.where(np.arange(w) % 2, 0xFF00, 0x00FF)
    tiles[4, 0] = 0x0001
    tiles[5, :w] = synth.uniform_u16(seed, w)
    return tiles


def h128_matrix():
    h = np.ones((1, 1))
    while h.shape[0] < 128:
        h = np.block([[h, h], [h, -h]])
    return h / np.sqrt(128.0)


def get_rows_fixture(ref):
    k, n, bits, cb, seed = 256, 384, 6, 2, 7007
    p = synth.packed_tiles(seed, k, n, bits)
    su, sv = synth.layer_scales(seed, k, n)
    records = synth.pack_records(p, su, sv, bits).view(np.uint8)
    gb = synth.group_bytes(bits)
    ids = np.array([0, n // 2, n - 1, 128, 5, 255, n - 1], dtype=np.int32)
    out = np.zeros((ids.size, k), dtype=np.float32)
    for r, i in enumerate(ids):
        for kb in range(k // 128):
            g = records[(i // 128 * (k // 128) + kb) * gb:][:gb]
            tiles = g[: 2048 * bits].view(np.uint16)
            gsu = g[2048 * bits: 2048 * bits + 256].view(np.float16)
            gsv = g[2048 * bits + 256: 2048 * bits + 512].view(np.float16)
            blk = ref.reconstruct(tiles, gsu, gsv, 128, 128, bits, cb)
            out[r, kb * 128:(kb + 1) * 128] = blk[:, i % 128].view(np.float16).astype(np.float32)
    np.savez(HERE / "get_rows.npz", meta=np.array([k, n, bits, cb, seed]), ids=ids, out=out,
             records_sha256=np.array(sha(records)))


def main():
    ref = Reference()
    only = sys.argv[1:]
    if only:
        for name in only:
            {"get_rows": get_rows_fixture}[name](ref)
        print("golden fixtures written to", HERE)
        return
    # 1. codebooks
    cbj = {}
    spots = list(range(0, 65536, 257)) + [65535]
    for cb in range(3):
        t = ref.codebook_table(cb)
        cbj[str(cb)] = {"sha256": sha(t.astype("<u2")), "states": spots, "values": [int(t[s]) for s in spots]}
    (HERE / "codebook.json").write_text(json.dumps(cbj, indent=1) + "\n")

    # 2. tiles
    packed = np.zeros((8, 3, 6, 128), dtype=np.uint16)
    decoded = np.zeros((8, 3, 6, 256), dtype=np.uint16)
    for bits in range(1, 9):
        for cb in range(3):
            tiles = edge_tiles(bits, 1000 * bits + cb)
            packed[bits - 1, cb] = tiles
            for t in range(6):
                decoded[bits - 1, cb, t] = ref.decode_tile(tiles[t, : 16 * bits], bits, cb).reshape(-1)
    np.savez(HERE / "tiles.npz", packed=packed, decoded=decoded)

    # 3. 256x384 matrices (the reference fixture geometry, tests/generate_cuda_fixtures.py:69-72)
    mats = []
    k, n = 256, 384
    probe = [0, 1, 17, 255, 384, 4095, 40000, k * n - 1]
    for bits in range(1, 9):
        for cb in range(3):
            seed = bits * 100 + cb
            p = synth.packed_tiles(seed, k, n, bits)
            su = (synth.uniform01(seed ^ 0x11, k) * 2 - 1).astype(np.float16)
            sv = (synth.uniform01(seed ^ 0x22, n) * 2 - 1).astype(np.float16)
            inner = ref.decode_inner(p, k, n, bits, cb)
            orig = ref.reconstruct(p, su, sv, k, n, bits, cb)
            mats.append({"bits": bits, "cb": cb, "seed": seed, "k": k, "n": n,
                         "packed_sha256": sha(p.astype("<u2")), "su_sha256": sha(su), "sv_sha256": sha(sv),
                         "inner_sha256": sha(inner.astype("<u2")), "original_sha256": sha(orig.astype("<u2")),
                         "probe": probe, "inner_probe": [int(inner.reshape(-1)[i]) for i in probe],
                         "original_probe": [int(orig.reshape(-1)[i]) for i in probe]})
    (HERE / "matrices.json").write_text(json.dumps(mats, indent=1) + "\n")

    # 4. hadamard
    vecs = [np.zeros(128, np.float32), np.eye(128, dtype=np.float32)[5], np.ones(128, np.float32),
            (synth.normal(77, 256) * 3).astype(np.float32)]
    hj = []
    for v in vecs:
        out = ref.hadamard128(v)
        hj.append({"input": v.view(np.uint32).tolist(), "output": out.view(np.uint32).tolist()})
    (HERE / "hadamard.json").write_text(json.dumps(hj) + "\n")

    # 5. layer: k=256, n=256, bits 4, mul1, 3 rows
    k, n, bits, cb, rows = 256, 256, 4, 2, 3
    p = synth.packed_tiles(4242, k, n, bits)
    su, sv = synth.layer_scales(4242, k, n)
    x = synth.activations(4243, rows, k)
    records = synth.pack_records(p, su, sv, bits)
    inner = ref.decode_inner(p, k, n, bits, cb).view(np.float16).astype(np.float64)
    H = h128_matrix()
    Hk = np.kron(np.eye(k // 128), H)
    Hn = np.kron(np.eye(n // 128), H)
    xh = (x.astype(np.float64) * su.astype(np.float64)) @ Hk
    y = ((xh @ inner) @ Hn) * sv.astype(np.float64)
    orig = ref.reconstruct(p, su, sv, k, n, bits, cb).view(np.float16).astype(np.float64)
    y_recon = x.astype(np.float64) @ orig
    np.savez(HERE / "layer.npz", records=records, x=x, y=y, y_from_reconstruct=y_recon,
             meta=np.array([k, n, bits, cb, rows]))

    # 6. EXL3REF1 fixtures
    for (bits, cb, k, n, seed) in [(4, 2, 128, 256, 9001), (3, 0, 128, 128, 9002)]:
        p = synth.packed_tiles(seed, k, n, bits)
        su = (synth.uniform01(seed ^ 0x11, k) * 2 - 1).astype(np.float16)
        sv = (synth.uniform01(seed ^ 0x22, n) * 2 - 1).astype(np.float16)
        inner = ref.decode_inner(p, k, n, bits, cb)
        orig = ref.reconstruct(p, su, sv, k, n, bits, cb)
        with open(HERE / f"k{bits}-cb{cb}-{k}x{n}.exl3ref", "wb") as f:
            f.write(b"EXL3REF1" + struct.pack("<4I", k, n, bits, cb))
            for a in (p.astype("<u2"), su.view("<u2"), sv.view("<u2"), inner.astype("<u2"), orig.astype("<u2")):
                f.write(np.ascontiguousarray(a).tobytes())
    # 7. GET_ROWS
    get_rows_fixture(ref)
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
