"""The model reader's host-side passes (csrc/exl3_model_format.cpp) and the
JSON reader (csrc/exl3_json.hpp) built with AddressSanitizer and
UndefinedBehaviorSanitizer (g++, no GPU code) and fed the reference reader
test's model, every malformed model of tests/test_model.py, randomly built
models, and mutated JSON text.  Any out-of-bounds access, leak or undefined
operation aborts the driver (-fno-sanitize-recover)."""
import copy
import json
import subprocess
from pathlib import Path

import pytest

from model_files import random_model, reference_case, write_model
from test_model import mutations

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "xiaomi-hexagon-exl3_amd" / "csrc"
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"]


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = tmp_path_factory.mktemp("san") / "model_format_check"
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", *SAN, "-Wall", "-Wextra", f"-I{CSRC}", "-o", str(exe),
                    str(ROOT / "tests" / "cpp" / "model_format_check.cpp"), str(CSRC / "exl3_model_format.cpp")],
                   check=True)
    return exe


def run(checker, args):
    r = subprocess.run([str(checker), *map(str, args)], capture_output=True, text=True, timeout=300,
                       env={"ASAN_OPTIONS": "detect_leaks=1", "UBSAN_OPTIONS": "print_stacktrace=1"})
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "Sanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-4000:]
    return r.stdout.splitlines()


def test_sanitized_reader_on_good_and_malformed_models(checker, tmp_path):
    dirs, expect = [], []
    good = tmp_path / "reference"
    good.mkdir()
    write_model(good, *reference_case())
    dirs.append(good)
    expect.append("OPEN")
    for i, (name, mutate) in enumerate(mutations()):
        d = tmp_path / f"bad{i}"
        d.mkdir()
        header, data, manifest = reference_case()
        write_model(d, *mutate(copy.deepcopy(header), bytes(data), copy.deepcopy(manifest)))
        dirs.append(d)
        expect.append("REJECT")
    # header-level damage: length past the file, garbage text, header not an object, truncated file
    for j, raw in enumerate((b"\xff" * 8, b"\x04\x00\x00\x00\x00\x00\x00\x00[1] ", b"\x06\x00\x00\x00\x00\x00\x00\x00{\"a\":",
                             b"\x01\x00")):
        d = tmp_path / f"raw{j}"
        d.mkdir()
        (d / "model.safetensors").write_bytes(raw)
        (d / "hexagon-exl3.json").write_text(json.dumps(reference_case()[2]))
        dirs.append(d)
        expect.append("REJECT")
    absent = tmp_path / "absent"
    dirs.append(absent)
    expect.append("REJECT")
    mats = [("model.layers.0.mlp.down_proj", 256, 128, 3, 0), ("model.layers.0.mlp.gate_proj", 128, 256, 5, 1),
            ("lm_head", 128, 384, 4, 2)]
    rnd = tmp_path / "random"
    rnd.mkdir()
    header, data, manifest, _ = random_model(90, mats, "lm_head")
    write_model(rnd, header, data, manifest)
    dirs.append(rnd)
    expect.append("OPEN")
    lines = run(checker, dirs)
    assert len(lines) == len(dirs)
    for line, want, d in zip(lines, expect, dirs):
        assert line.startswith(f"{want} {d}"), line
    assert lines[0].split()[2:] == ["4", "8708", "4", "2", "1"]          # tensors, payload, bits, mul1, matrices
    assert lines[-1].split()[2:] == ["11", str(len(data)), "4", "2", "3"]


def test_sanitized_json_reader_fuzz(checker, tmp_path):
    header, data, manifest = reference_case()
    for name, doc in (("header.json", header), ("manifest.json", manifest)):
        f = tmp_path / name
        f.write_text(json.dumps(doc))
        out = run(checker, ["--json-fuzz", 1234, 4000, f])
        assert out[-1].startswith("FUZZ"), out
        parsed, rejected = map(int, out[-1].split()[1:])
        assert parsed + rejected == 4000 and rejected > 0
