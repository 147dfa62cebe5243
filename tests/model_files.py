"""Writes EXL3 deployment-model directories (model.safetensors + hexagon-exl3.json)
the way the reference's tests/test_model_reader.cpp:23-46 does, for the model
reader tests."""
import json
import struct

import numpy as np

import synth


def write_model(directory, header, data, manifest):
    text = json.dumps(header)
    text += " " * ((8 - len(text) % 8) % 8)
    with open(directory / "model.safetensors", "wb") as f:
        f.write(struct.pack("<Q", len(text)))
        f.write(text.encode())
        f.write(bytes(data))
    (directory / "hexagon-exl3.json").write_text(json.dumps(manifest))


def reference_case():
    """test_model_reader.cpp:23-37: a 128x128 4-bit zero trellis head, su = sv = 1, mul1 marker"""
    header = {
        "lm_head.trellis": {"dtype": "I16", "shape": [8, 8, 64], "data_offsets": [0, 8192]},
        "lm_head.suh": {"dtype": "F16", "shape": [128], "data_offsets": [8192, 8448]},
        "lm_head.svh": {"dtype": "F16", "shape": [128], "data_offsets": [8448, 8704]},
        "lm_head.mul1": {"dtype": "I32", "shape": [], "data_offsets": [8704, 8708]},
    }
    manifest = {"format": "hexagon-exl3", "version": 1, "kv_cache": "f16",
                "reference_parameter_count": 16384, "weight_payload_bytes": 8708,
                "input_embedding": {"type": "tied_linear", "source": "lm_head", "basis": "original",
                                    "token_axis": 1, "hidden_size": 128, "vocab_size": 128}}
    data = bytearray(8708)
    for i in range(8192, 8704, 2):
        data[i + 1] = 0x3C
    data[8704:8708] = struct.pack("<I", 0x83DCD12D)
    return header, data, manifest


MARKERS = {2: ("mul1", 0x83DCD12D), 1: ("mcg", 0xCBAC1FED)}


def random_model(seed, matrices, head):
    """matrices: [(prefix, k, n, bits, cb)]; head: the prefix of the tied head.
    Returns header, data, manifest and {prefix: (packed, su, sv)}."""
    header, chunks, parts, off, params = {}, [], {}, 0, 0
    for i, (prefix, k, n, bits, cb) in enumerate(matrices):
        p = synth.packed_tiles(seed + i, k, n, bits)
        su, sv = synth.layer_scales(seed + i, k, n)
        parts[prefix] = (p, su, sv)
        params += k * n
        tensors = [(".trellis", "I16", [k // 16, n // 16, 16 * bits], p.astype("<u2").tobytes()),
                   (".suh", "F16", [k], su.astype("<f2").tobytes()),
                   (".svh", "F16", [n], sv.astype("<f2").tobytes())]
        if cb in MARKERS:
            tensors.append(("." + MARKERS[cb][0], "I32", [], struct.pack("<I", MARKERS[cb][1])))
        for suffix, dtype, shape, raw in tensors:
            header[prefix + suffix] = {"dtype": dtype, "shape": shape, "data_offsets": [off, off + len(raw)]}
            chunks.append(raw)
            off += len(raw)
    hk, hn = next((k, n) for prefix, k, n, _, _ in matrices if prefix == head)
    manifest = {"format": "hexagon-exl3", "version": 1, "kv_cache": "f16",
                "reference_parameter_count": params, "weight_payload_bytes": off,
                "input_embedding": {"type": "tied_linear", "source": head, "basis": "original",
                                    "token_axis": 1, "hidden_size": hk, "vocab_size": hn}}
    return header, b"".join(chunks), manifest, parts
