"""exl3::Model, the deployment-model reader (src/exl3_model.cpp:79-187), through
the C-ABI: the reference's own reader test (tests/test_model_reader.cpp:23-73)
and further malformed inputs on the CPU; embeddings and record uploads on the GPU
against the oracle."""
import copy
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

import conftest
import synth
from model_files import random_model, reference_case, write_model


def amd_lib():
    return conftest.load_amd()


def open_or_reason(d):
    amd = amd_lib()
    try:
        return amd.Model(d), None
    except amd.Exl3Error as e:
        return None, str(e)


def test_reference_reader_case_opens(tmp_path):
    header, data, manifest = reference_case()
    write_model(tmp_path, header, data, manifest)
    m, why = open_or_reason(tmp_path)
    assert m is not None, why
    with m:
        # test_model_reader.cpp:49
        assert m.tensor_count == 4 and m.payload_bytes == 8708
        assert m.hidden_size == 128 and m.vocab_size == 128
        assert m.bits_per_weight == pytest.approx(8708 * 8 / 16384)
        assert m.matrices() == [("lm_head", 4, 2, 128, 128)]


def mutations():
    """(name, mutate(header, data, manifest)) -> each must be rejected"""
    def set_(path, value, which):
        def f(h, d, m):
            tgt = {"h": h, "m": m}[which]
            for key in path[:-1]:
                tgt = tgt[key]
            tgt[path[-1]] = value
            return h, d, m
        return f
    def drop(path, which):
        def f(h, d, m):
            tgt = {"h": h, "m": m}[which]
            for key in path[:-1]:
                tgt = tgt[key]
            del tgt[path[-1]]
            return h, d, m
        return f
    def truncate(h, d, m):
        return h, d[:-1], m
    def add_mcg(h, d, m):
        h["lm_head.mcg"] = {"dtype": "I32", "shape": [], "data_offsets": [8708, 8712]}
        m["weight_payload_bytes"] = 8712
        return h, d + struct.pack("<I", 0xCBAC1FED), m
    def bad_mul1(h, d, m):
        d = bytearray(d)
        d[8704:8708] = struct.pack("<I", 0x12345678)
        return h, d, m
    return [
        # the four rejections of tests/test_model_reader.cpp:67-72
        ("budget: parameter count 1", set_(["reference_parameter_count"], 1, "m")),
        ("overlapping spans", set_(["lm_head.suh", "data_offsets"], [8190, 8446], "h")),
        ("negative dimension", set_(["lm_head.suh", "shape"], [-128], "h")),
        ("truncated payload", truncate),
        # further checks of src/exl3_model.cpp:79-156
        ("zero dimension", set_(["lm_head.suh", "shape"], [0], "h")),
        ("real dimension", set_(["lm_head.suh", "shape"], [128.0], "h")),
        ("unsupported dtype", set_(["lm_head.suh", "dtype"], "F64", "h")),
        ("span length != shape", set_(["lm_head.svh", "shape"], [64], "h")),
        ("offset pair of 3", set_(["lm_head.svh", "data_offsets"], [8448, 8704, 8704], "h")),
        ("gap in payload", set_(["lm_head.svh", "data_offsets"], [8450, 8706], "h")),
        ("payload bytes mismatch", set_(["weight_payload_bytes"], 8700, "m")),
        ("manifest format", set_(["format"], "exl3", "m")),
        ("manifest version", set_(["version"], 2, "m")),
        ("kv cache", set_(["kv_cache"], "q8", "m")),
        ("embedding type", set_(["input_embedding", "type"], "linear", "m")),
        ("token axis", set_(["input_embedding", "token_axis"], 0, "m")),
        ("hidden size not /128", set_(["input_embedding", "hidden_size"], 96, "m")),
        ("missing source tensor", set_(["input_embedding", "source"], "head", "m")),
        ("missing manifest key", drop(["kv_cache"], "m")),
        ("trellis dtype", set_(["lm_head.trellis", "dtype"], "F16", "h")),
        ("trellis shape", set_(["lm_head.trellis", "shape"], [8, 4, 128], "h")),
        ("ambiguous codebook", add_mcg),
        ("mul1 multiplier", bad_mul1),
    ]


@pytest.mark.parametrize("name,mutate", mutations(), ids=[m[0] for m in mutations()])
def test_malformed_models_rejected(tmp_path, name, mutate):
    header, data, manifest = reference_case()
    header, data, manifest = mutate(copy.deepcopy(header), bytes(data), copy.deepcopy(manifest))
    write_model(tmp_path, header, data, manifest)
    m, why = open_or_reason(tmp_path)
    assert m is None, name
    assert why


def test_header_length_and_missing_files(tmp_path):
    header, data, manifest = reference_case()
    write_model(tmp_path, header, data, manifest)
    raw = bytearray((tmp_path / "model.safetensors").read_bytes())
    raw[0:8] = struct.pack("<Q", len(raw))            # header longer than the file
    (tmp_path / "model.safetensors").write_bytes(bytes(raw))
    assert open_or_reason(tmp_path)[0] is None
    write_model(tmp_path, header, data, manifest)
    (tmp_path / "hexagon-exl3.json").unlink()
    assert open_or_reason(tmp_path)[0] is None
    assert open_or_reason(tmp_path / "absent")[0] is None


def test_codebook_markers_and_matrix_inventory(tmp_path):
    mats = [("model.layers.0.mlp.down_proj", 256, 128, 3, 0), ("model.layers.0.mlp.gate_proj", 128, 256, 5, 1),
            ("lm_head", 128, 384, 4, 2)]     # 4.0 bits per weight on average: within the 5.0 budget
    header, data, manifest, _ = random_model(90, mats, "lm_head")
    write_model(tmp_path, header, data, manifest)
    m, why = open_or_reason(tmp_path)
    assert m is not None, why
    with m:
        assert m.tensor_count == 3 * 3 + 2            # the 3inst matrix has no marker
        assert sorted(m.matrices()) == sorted((p, b, c, k, n) for p, k, n, b, c in mats)
        assert m.hidden_size == 128 and m.vocab_size == 384


# ---- GPU ------------------------------------------------------------------------

@pytest.mark.gpu
def test_embedding_known_answer(tmp_path, amd, oracle):
    # test_model_reader.cpp:50-59
    header, data, manifest = reference_case()
    write_model(tmp_path, header, data, manifest)
    with amd.Model(tmp_path) as m:
        row0, row1 = m.embedding(0), m.embedding(1)
        assert np.array_equal(row0, m.embedding(0))
        code = oracle.L.orc_half_to_float(oracle.L.orc_decode_codebook(0, 2))
        assert row0[0] == oracle.L.orc_float_to_half(code * 128)
        assert np.all(row0[1:].view(np.float16) == 0) and np.all(row1.view(np.float16) == 0)
        with pytest.raises(amd.Exl3Error):
            m.embedding(128)


@pytest.mark.gpu
def test_embedding_matches_reconstruct_across_groups(tmp_path, amd, oracle):
    # a 4-bit mcg head of 20 token groups: more groups than the 16-entry cache holds
    k, n = 256, 128 * 20
    header, data, manifest, parts = random_model(91, [("lm_head", k, n, 4, 1)], "lm_head")
    write_model(tmp_path, header, data, manifest)
    p, su, sv = parts["lm_head"]
    full = oracle.reconstruct(p, su, sv, k, n, 4, 1)
    tokens = [0, 5, 130, 127, 2559, 1000] + [128 * g + g for g in range(20)] + [0, 5, 2559]
    with amd.Model(tmp_path) as m:
        for t in tokens:
            assert np.array_equal(m.embedding(t), full[:, t]), t


@pytest.mark.gpu
def test_upload_records_feed_the_layer(tmp_path, amd, oracle):
    import torch
    from gpu_util import assert_layer_close
    mats = [("model.layers.0.mlp.down_proj", 256, 128, 3, 0), ("lm_head", 128, 384, 4, 2)]
    header, data, manifest, parts = random_model(92, mats, "lm_head")
    write_model(tmp_path, header, data, manifest)
    with amd.Model(tmp_path) as m:
        inventory = m.matrices()
        for idx, (prefix, bits, cb, k, n) in enumerate(inventory):
            p, su, sv = parts[prefix]
            rec = m.upload_records(idx)
            torch.cuda.synchronize()
            want = synth.pack_records(p, su, sv, bits).view(np.uint8)
            assert np.array_equal(rec.cpu().numpy(), want), prefix
            x = synth.activations(93 + idx, 3, k)
            y = amd.mul_mat(rec, bits, k, n, torch.from_numpy(x).cuda(), codebook=cb).cpu().numpy()
            assert_layer_close(y, oracle.mul_mat(want, bits, cb, k, n, x), what=prefix)


@pytest.mark.gpu
def test_cpp_model_api_program(tmp_path):
    """tests/cpp/test_model_api.cpp: exl3::Model through its C++ class, as the
    reference's tests/test_model_reader.cpp drives its own (known-answer tied
    embedding, row cache, token bound, four rejections)."""
    exe = Path(__file__).resolve().parent / "cpp" / "test_model_api"
    assert exe.exists(), "tests/cpp/test_model_api is built by __graft_entry__.build()"
    r = subprocess.run([str(exe), str(tmp_path)], capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0 and "PASS" in r.stdout


def _with_embedding_table(header, data, manifest, rows, groups, bits, signs_cols=256, trellis_dtype="I16",
                          signs_dtype="F16", words=None):
    """adds a row-coded table emb.trellis [rows, groups * words] + emb.signs [groups, 256]
    (tools/inspect_model.py:78-90) to a model and fixes the manifest's payload"""
    words = 16 * bits + 1 if words is None else words
    off = len(data)
    width = {"I16": 2, "F16": 2, "F32": 4}
    tb = rows * groups * words * width[trellis_dtype]
    sb = groups * signs_cols * width[signs_dtype]
    header = dict(header)
    header["emb.trellis"] = {"dtype": trellis_dtype, "shape": [rows, groups * words], "data_offsets": [off, off + tb]}
    header["emb.signs"] = {"dtype": signs_dtype, "shape": [groups, signs_cols], "data_offsets": [off + tb, off + tb + sb]}
    manifest = dict(manifest)
    manifest["weight_payload_bytes"] = off + tb + sb
    manifest["reference_parameter_count"] = 10 ** 6     # keep the 5.0 bpw budget
    return header, bytes(data) + bytes(tb + sb), manifest


def test_row_coded_embedding_tables(tmp_path):
    """Row-coded EXL3 embedding tables are listed with their geometry and
    rejected, with the reference audit's messages, when malformed
    (tools/inspect_model.py:78-90); the model itself still opens."""
    amd = amd_lib()
    cases = [  # (rows, groups, bits, kwargs, expected reason or None)
        (6, 3, 4, {}, None),
        (2, 1, 1, {}, None),
        (4, 2, 8, {}, None),
        (4, 2, 4, {"signs_cols": 128}, "Invalid EXL3 embedding: emb.trellis"),
        (4, 2, 4, {"trellis_dtype": "F16"}, "Invalid EXL3 embedding: emb.trellis"),
        (4, 2, 4, {"signs_dtype": "F32"}, "Invalid EXL3 embedding: emb.trellis"),
        (4, 2, 4, {"words": 16 * 4}, "Invalid EXL3 embedding bitrate: emb.trellis"),    # no header word
        (4, 2, 9, {}, "Invalid EXL3 embedding bitrate: emb.trellis"),                    # 9 bits
        (4, 1, 0, {"words": 1}, "Invalid EXL3 embedding bitrate: emb.trellis"),          # 0 bits
    ]
    for i, (rows, groups, bits, kw, reason) in enumerate(cases):
        d = tmp_path / f"m{i}"
        d.mkdir()
        write_model(d, *_with_embedding_table(*reference_case(), rows, groups, bits, **kw))
        m, why = open_or_reason(d)
        assert m is not None, (i, why)
        with m:
            if reason is None:
                assert m.embedding_tables() == [("emb", rows, groups, bits, groups * 256)], i
                assert m.matrices() == [("lm_head", 4, 2, 128, 128)]   # the table is not a matrix
            else:
                with pytest.raises(amd.Exl3Error) as e:
                    m.embedding_tables()
                assert reason in str(e.value), (i, str(e.value))
    # group count that does not divide the code width
    d = tmp_path / "groups"
    d.mkdir()
    header, data, manifest = _with_embedding_table(*reference_case(), 4, 3, 4)
    header["emb.trellis"]["shape"] = [4, 3 * 65 + 1]
    header["emb.trellis"]["data_offsets"][1] += 8
    header["emb.signs"]["data_offsets"] = [o + 8 for o in header["emb.signs"]["data_offsets"]]
    manifest["weight_payload_bytes"] += 8
    write_model(d, header, bytes(data) + bytes(8), manifest)
    with amd.Model(d) as m:
        with pytest.raises(amd.Exl3Error) as e:
            m.embedding_tables()
        assert "Invalid EXL3 embedding groups: emb.trellis" in str(e.value)
    with amd.Model(tmp_path / "m0") as m:   # the reference test's model has none
        pass
    d = tmp_path / "plain"
    d.mkdir()
    write_model(d, *reference_case())
    with amd.Model(d) as m:
        assert m.embedding_tables() == []
