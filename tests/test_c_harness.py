"""The plain-C side of the boundary: include/qff/qff.h compiles as strict C99
(the Swift importer reads it as C), the Swift module map points at it, and a
C program that links libqff_hip.so and calls it with no C++ or torch in the
process (tests/c_harness/qff_harness.c) gets the oracle's results on the GPU."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qff", "qff.h")
MODULEMAP = os.path.join(ROOT, "swift", "QwenFieldfareHIP", "module.modulemap")
HARNESS = os.path.join(ROOT, "tests", "c_harness", "build", "qff_harness")


def test_header_is_strict_c99(tmp_path):
    src = tmp_path / "use_qff.c"
    src.write_text('#include "qff/qff.h"\n'
                   "int main(void) { qff_ctx_cfg c = {1, 2, 3}; qff_stream_t s = 0;"
                   " return c.max_batch + (int)QFF_BF16 + (s == 0); }\n")
    for std in ("c99", "c11"):
        r = subprocess.run(["gcc", f"-std={std}", "-pedantic", "-Wall", "-Wextra", "-Werror", "-fsyntax-only",
                            "-I", os.path.join(ROOT, "include"), str(src)], capture_output=True, text=True)
        assert r.returncode == 0, r.stderr


def test_module_map_names_the_header_and_library():
    text = re.sub(r"//[^\n]*", "", open(MODULEMAP).read())
    m = re.search(r"module\s+QwenFieldfareHIP\s*\[system\]\s*\{(.*)\}", text, flags=re.S)
    assert m, "module QwenFieldfareHIP [system] { ... }"
    body = m.group(1)
    hdr = re.search(r'header\s+"([^"]+)"', body).group(1)
    assert os.path.samefile(os.path.join(os.path.dirname(MODULEMAP), hdr), HEADER)
    assert re.search(r'link\s+"qff_hip"', body)
    assert "export *" in body


def test_harness_source_builds_warning_free(tmp_path):
    """The harness compiles with -Wall -Wextra -Werror (the binary the GPU
    test runs is built by __graft_entry__.build())."""
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-fsyntax-only", "-D__HIP_PLATFORM_AMD__",
                        "-I", os.path.join(ROOT, "include"), "-I", "/opt/rocm/include",
                        os.path.join(ROOT, "tests", "c_harness", "qff_harness.c")], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


@pytest.mark.gpu
def test_c_harness_matches_oracle_on_gpu():
    print("c harness (qff_deltanet_decode, qff_gqa_decode, error paths)", flush=True)
    assert os.access(HARNESS, os.X_OK), "build the harness first (__graft_entry__.build())"
    r = subprocess.run([HARNESS], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0 and "qff_harness: OK" in r.stdout
