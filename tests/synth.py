"""Seeded synthetic inputs for the EXL3 linear layer (tests, fixtures, bench).

Counter-based splitmix64 in numpy: element i of stream (seed) is
mix64(seed + (i + 1) * 0x9e3779b97f4a7c15), so any prefix of a stream is
reproducible bit for bit on any machine.  Normal draws use Box-Muller in
float64 and are then rounded to fp16.
"""
import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed, count, offset=0):
    i = np.arange(offset + 1, offset + count + 1, dtype=np.uint64)
    z = np.uint64(seed) + i * GAMMA
    z = (z ^ (z >> np.uint64(30))) * M1
    z = (z ^ (z >> np.uint64(27))) * M2
    return z ^ (z >> np.uint64(31))


def uniform_u16(seed, count):
    return (splitmix64(seed, count) >> np.uint64(48)).astype(np.uint16)


def uniform01(seed, count):
    return (splitmix64(seed, count) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def normal(seed, count, sigma=1.0):
    half = (count + 1) // 2
    u = uniform01(seed, 2 * half)
    r = np.sqrt(-2.0 * np.log1p(-u[0::2]))
    t = 2.0 * np.pi * u[1::2]
    z = np.concatenate([r * np.cos(t), r * np.sin(t)])[:count]
    return z * sigma


def signs(seed, count):
    return np.where(splitmix64(seed, count) >> np.uint64(63), -1.0, 1.0)


def packed_tiles(seed, k, n, bits):
    """Upstream tile grid [k/16][n/16][16*bits] of uniform u16."""
    return uniform_u16(seed, (k // 16) * (n // 16) * 16 * bits).reshape(k // 16, n // 16, 16 * bits)


def layer_scales(seed, k, n):
    """su = +-1, sv = +-U(0.5, 1.5)/sqrt(k), both fp16 (the layer workload recipe)."""
    su = signs(seed ^ 0x5555, k).astype(np.float16)
    mag = 0.5 + uniform01(seed ^ 0xAAAA, n)
    sv = (signs(seed ^ 0x3333, n) * mag / np.sqrt(k)).astype(np.float16)
    return su, sv


def activations(seed, rows, k, sigma=1.0):
    return normal(seed, rows * k, sigma).astype(np.float16).reshape(rows, k)


def pack_records(packed, su, sv, bits):
    """Upstream tiles + scales -> 128x128 group records (bytes), the layout of
    include/exl3-block.h; tests/test-exl3-graph.cpp:37-45."""
    kt, nt, w = packed.shape
    k, n = kt * 16, nt * 16
    assert w == 16 * bits and k % 128 == 0 and n % 128 == 0
    tiles = packed.reshape(k // 128, 8, n // 128, 8, 16 * bits).transpose(2, 0, 1, 3, 4)
    tiles = tiles.reshape(n // 128, k // 128, 1024 * bits)
    rec = np.empty((n // 128, k // 128, 1024 * bits + 256), dtype=np.uint16)
    rec[:, :, : 1024 * bits] = tiles
    rec[:, :, 1024 * bits : 1024 * bits + 128] = su.view(np.uint16).reshape(1, k // 128, 128)
    rec[:, :, 1024 * bits + 128 :] = sv.view(np.uint16).reshape(n // 128, 1, 128)
    return rec.reshape(-1)


def group_bytes(bits):
    return 2048 * bits + 512


def c2_matrices():
    """The 151 weight matrices (k in, n out) of the synthetic 2B hybrid model of the
    dequant sweep: 24 MLP blocks (gate, up 2048->6144, down 6144->2048), 6 full
    attention blocks (q 2048->2048, k and v 2048->512, o 2048->2048), 18
    linear-attention blocks (2048->2048, 2048->2048, 2048->512) and the vocabulary
    head 2048->151936."""
    mats = []
    for _ in range(24):
        mats += [(2048, 6144), (2048, 6144), (6144, 2048)]
    for _ in range(6):
        mats += [(2048, 2048), (2048, 512), (2048, 512), (2048, 2048)]
    for _ in range(18):
        mats += [(2048, 2048), (2048, 2048), (2048, 512)]
    mats.append((2048, 151936))
    return mats


def c2_bits(mats):
    """Bits per matrix from {2..6} by seed, redrawn until the weight-weighted mean
    is <= 5.0 bits per weight."""
    w = np.array([k * n for k, n in mats], dtype=np.float64)
    for attempt in range(1000):
        b = (splitmix64(2222 + attempt, len(mats)) % np.uint64(5)).astype(int) + 2
        if float(np.sum(w * b) / np.sum(w)) <= 5.0:
            return b
    raise RuntimeError("no bit draw met the 5.0 bpw bound")
