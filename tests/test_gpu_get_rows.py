"""GPU GET_ROWS parity (ggml_exl3_get_rows, src/exl3-ggml.cpp:19-49): every value
bit-exact with the oracle and with the golden rows made by the compiled
reference codec; id patterns of tests/test-exl3-graph.cpp:106-134."""
from pathlib import Path

import numpy as np
import pytest

import synth
from gpu_util import dev

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"


def ids_tensor(ids):
    import torch
    return torch.from_numpy(np.ascontiguousarray(ids, dtype=np.int32)).cuda()


def test_get_rows_golden(amd):
    d = np.load(GOLD / "get_rows.npz")
    k, n, bits, cb, seed = (int(v) for v in d["meta"])
    print(f"  get_rows golden {k}x{n} bits={bits}", flush=True)
    p = synth.packed_tiles(seed, k, n, bits)
    su, sv = synth.layer_scales(seed, k, n)
    rec = dev(synth.pack_records(p, su, sv, bits).view(np.uint8))
    out = amd.get_rows(rec, bits, k, n, ids_tensor(d["ids"]), codebook=cb).cpu().numpy()
    assert np.array_equal(out.view(np.uint32), d["out"].view(np.uint32))


@pytest.mark.parametrize("bits,cb", [(2, 2), (4, 2), (6, 1), (3, 0)])
def test_get_rows_matches_oracle(amd, oracle, bits, cb):
    import torch
    k, n = 512, 640
    print(f"  get_rows {k}x{n} bits={bits} cb={cb}", flush=True)
    p = synth.packed_tiles(50 + bits, k, n, bits)
    su, sv = synth.layer_scales(50 + bits, k, n)
    rec_h = synth.pack_records(p, su, sv, bits).view(np.uint8)
    rec = dev(rec_h)
    ids = np.array([0, n // 2, n - 1, 1, 127, 128, 333, 0], dtype=np.int32)
    want = oracle.get_rows(rec_h, bits, cb, k, n, ids)
    got32 = amd.get_rows(rec, bits, k, n, ids_tensor(ids), codebook=cb).cpu().numpy()
    assert np.array_equal(got32.view(np.uint32), want.view(np.uint32))
    got16 = amd.get_rows(rec, bits, k, n, ids_tensor(ids), codebook=cb, out_dtype=torch.float16).cpu().numpy()
    assert np.array_equal(got16.view(np.uint16), want.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("count", [1, 7])
def test_get_rows_vocab_head(amd, oracle, count):
    # tied embedding of the 2B model's head: k = 2048 hidden, a vocabulary slice, 6 bits;
    # ids as tests/test-exl3-graph.cpp:113: n - 1 for one row, else 0, n / 2, n - 1 cycling
    k, n, bits = 2048, 151936 // 8 // 128 * 128, 6
    print(f"  get_rows head {k}x{n} count={count}", flush=True)
    p = synth.packed_tiles(606, k, n, bits)
    su, sv = synth.layer_scales(606, k, n)
    rec_h = synth.pack_records(p, su, sv, bits).view(np.uint8)
    ids = np.array([n - 1] if count == 1 else [(0, n // 2, n - 1)[r % 3] for r in range(count)], dtype=np.int32)
    got = amd.get_rows(dev(rec_h), bits, k, n, ids_tensor(ids)).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), oracle.get_rows(rec_h, bits, 2, k, n, ids).view(np.uint32))


def test_get_rows_strides_bad_ids_and_empty(amd, oracle):
    import torch
    k, n, bits = 256, 384, 4
    p = synth.packed_tiles(77, k, n, bits)
    su, sv = synth.layer_scales(77, k, n)
    rec_h = synth.pack_records(p, su, sv, bits).view(np.uint8)
    rec = dev(rec_h)
    ids = np.array([5, n, 200, -3], dtype=np.int32)
    big = torch.full((4, k + 64), 7.0, dtype=torch.float32, device="cuda")
    out = big[:, :k]
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    amd.get_rows(rec, bits, k, n, ids_tensor(ids), out=out, bad_ids=flag)
    o = big.cpu().numpy()
    want = oracle.get_rows(rec_h, bits, 2, k, n, ids[[0, 2]])
    assert np.array_equal(o[[0, 2], :k], want)
    assert np.all(np.isnan(o[[1, 3], :k]))
    assert np.all(o[:, k:] == 7.0)                      # the padding past each row is untouched
    assert int(flag.item()) == 1
    flag.zero_()
    amd.get_rows(rec, bits, k, n, ids_tensor(ids[[0, 2]]), bad_ids=flag)
    torch.cuda.synchronize()
    assert int(flag.item()) == 0
    empty = amd.get_rows(rec, bits, k, n, ids_tensor(np.zeros(0, np.int32)))
    assert empty.shape == (0, k)
    L = amd.lib()
    assert L.exl3_hip_get_rows(None, 4, 2, 128, 128, None, 1, None, 0, 128, None, None) == 1
