"""The C-ABI library loads and exports every entry point include/qff/qff.h
declares, and the host-side argument checks that need no GPU behave. No
compute call runs here (this container has no GPU)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qff", "qff.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(qff_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_expected_surface():
    fns = declared_functions()
    for name in ("qff_ctx_create", "qff_ctx_destroy", "qff_workspace_size", "qff_status_string",
                 "qff_version", "qff_q4_dequant", "qff_q4_matmul", "qff_q4_matmul_parts",
                 "qff_q4_norm_matmul_parts", "qff_q8_dequant", "qff_router_top8", "qff_deltanet_decode",
                 "qff_deltanet_prefill", "qff_gqa_decode", "qff_gqa_prefill", "qff_kv_append",
                 "qff_attention_gate"):
        assert name in fns


def test_library_exports_every_declared_symbol():
    import qff
    from qff._lib import SIGNATURES
    L = qff.lib()
    for name in declared_functions():
        assert hasattr(L, name), f"{name} missing from {qff.LIB_PATH}"
        assert name in SIGNATURES, f"{name} has no ctypes signature"


def test_status_strings_and_version():
    import qff
    L = qff.lib()
    assert L.qff_status_string(0) == b"ok"
    assert L.qff_status_string(-4) == b"request exceeds the context workspace"
    assert L.qff_status_string(12345) == b"unknown status"
    assert L.qff_version() >= 1


def test_workspace_size_and_argument_checks_without_gpu():
    import qff
    from qff._lib import CtxCfg
    L = qff.lib()
    n = ctypes.c_size_t()
    assert L.qff_workspace_size(None, ctypes.byref(n)) == 0 and n.value > 0
    small = CtxCfg(1, 1024, 1)
    m = ctypes.c_size_t()
    assert L.qff_workspace_size(ctypes.byref(small), ctypes.byref(m)) == 0
    assert 0 < m.value < n.value
    assert L.qff_workspace_size(ctypes.byref(CtxCfg(-1, 0, 0)), ctypes.byref(m)) == -1
    assert L.qff_workspace_size(None, None) == -1
    # null context / outputs are rejected before any HIP call
    assert L.qff_ctx_create(None, 0, None) == -1
    assert L.qff_ctx_destroy(None) == -1
    N = None
    assert L.qff_deltanet_decode(N, N, N, N, N, 1, N, N, N, N, N, 1, 1) == -1
    assert L.qff_gqa_decode(N, N, N, N, N, N, 1, N, N, N, N, 1, 1, 16) == -1
    assert L.qff_q4_matmul(N, N, N, N, N, 2, N, 1, N, 0, 64, 64, 1) == -1
    assert L.qff_q4_matmul_parts(N, N, N, 1, 2, N, 1, 64, 1) == -1
    from qff._lib import Q4Part
    parts = (Q4Part * 9)()
    assert L.qff_q4_matmul_parts(N, N, parts, 9, 2, N, 1, 64, 1) == -1   # null ctx and too many parts
    assert L.qff_q4_norm_matmul_parts(N, N, N, 1, 2, N, 1, N, 0, 1e-6, 64, 1) == -1
    assert L.qff_q8_dequant(N, N, N, N, N, 1, N, 64, 64) == -1
    assert L.qff_router_top8(N, N, N, N, N, 1, N, 0, N, N, N, 256, 2048, 1) == -1


def test_product_has_no_cpu_fallback():
    """The product package never imports the oracle."""
    pkg = os.path.join(ROOT, "qwen-fieldfare_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".hpp", ".cpp", ".h")):
                src = open(os.path.join(dirpath, f)).read()
                assert not re.search(r"(from|import)\s+oracle|qff_oracle|libqff_oracle", src), f


def test_parameter_structs_match_the_header(tmp_path):
    """The ctypes mirrors of the header's parameter blocks have the C
    layout: a C program built against include/qff/qff.h prints each
    struct's size and every field's offset, and the ctypes classes must
    agree field for field (a field added on one side only would shift the
    others silently)."""
    import subprocess
    import sys
    sys.path.insert(0, os.path.join(ROOT, "qwen-fieldfare_amd"))
    from qff import _lib
    mirrors = {"qff_ctx_cfg": _lib.CtxCfg, "qff_q4_part": _lib.Q4Part,
               "qff_deltanet_params": _lib.DeltaNetParams, "qff_gqa_params": _lib.GqaParams}
    lines = ["#include <stddef.h>", "#include <stdio.h>", '#include "qff/qff.h"', "int main(void) {"]
    for cname, py in mirrors.items():
        lines.append(f'    printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in py._fields_:
            lines.append(f'    printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines += ["    return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    r = subprocess.run(["gcc", "-std=c99", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROOT, "include"),
                        "-o", str(exe), str(src)], capture_output=True, text=True)
    if r.returncode != 0:
        pytest.skip("no C compiler for the layout probe: " + r.stderr[-200:])
    got = dict(line.rsplit(" ", 1) for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                              check=True).stdout.splitlines())
    for cname, py in mirrors.items():
        assert int(got[f"{cname} size"]) == ctypes.sizeof(py), cname
        for fname, _ in py._fields_:
            assert int(got[f"{cname} {fname}"]) == getattr(py, fname).offset, (cname, fname)
