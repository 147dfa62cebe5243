"""CPU checks of the record header include/exl3-block.h and of source
compatibility with the reference's headers.

* tests/cpp/test_block_planners.c (plain C11, gcc) checks the record helpers
  and the Hexagon VTCM planners the header keeps: hand-computed plans and the
  invariants the reference's codec test requires of every plan
  (tests/test_codec.cpp:33-57 of the reference).
* The reference's own codec test, tests/test_codec.cpp, compiles against this
  repository's include/ and links with libexl3_hip.so (compile and link only
  here; running it needs the GPU, see tests/test_gpu_codec.py).  Skipped where
  the reference checkout is absent."""
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
REF = Path("/root/reference")
PKG = ROOT / "xiaomi-hexagon-exl3_amd"


def test_block_header_planners(tmp_path):
    exe = tmp_path / "test_block_planners"
    subprocess.run(["gcc", "-std=c11", "-O2", "-Wall", "-Wextra", "-Werror", "-pedantic", f"-I{ROOT / 'include'}",
                    "-o", str(exe), str(ROOT / "tests" / "cpp" / "test_block_planners.c")], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "PASS" in r.stdout


def test_block_header_compiles_as_cxx(tmp_path):
    src = tmp_path / "inc.cpp"
    src.write_text('#include "exl3-block.h"\n#include "exl3_codec.h"\n'
                   "int main() { return (int) exl3_row_chunk(4, 2048, 4, 262144) - 9; }\n")
    exe = tmp_path / "inc"
    subprocess.run(["g++", "-std=c++17", "-Wall", "-Wextra", "-Werror", f"-I{ROOT / 'include'}", "-o", str(exe),
                    str(src)], check=True)
    assert subprocess.run([str(exe)]).returncode == 0


@pytest.mark.skipif(not (REF / "tests" / "test_codec.cpp").exists(), reason="reference checkout absent")
def test_reference_codec_test_builds_against_include(tmp_path):
    exe = tmp_path / "test_codec_hip"
    r = subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Wextra", f"-I{ROOT / 'include'}", "-o", str(exe),
                        str(REF / "tests" / "test_codec.cpp"), f"-L{PKG}", "-lexl3_hip", "-L/opt/rocm/lib",
                        "-Wl,-rpath-link,/opt/rocm/lib"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    syms = subprocess.run(["nm", "-C", str(exe)], capture_output=True, text=True, check=True).stdout
    # every codec function the reference test calls resolves to this library
    for name in ("exl3::decode_codebook", "exl3::decode_tile", "exl3::hadamard128", "exl3::float_to_half",
                 "exl3::half_to_float", "exl3::decode_inner_slice"):
        assert name in syms, name
