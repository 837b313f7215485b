"""The drop-in boundary: liblaya.so loads on a machine without a GPU and exports every entry point
include/*.h declares; laya_api.h declares exactly the reference's ten entry points
(src/laya_api.h:5-19 of the reference).  No compute call is made here."""
import ctypes
import os
import re

import pytest

from layamd_amd import engine as le

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REFERENCE_ABI = ["laya_create", "laya_forward_batch", "laya_forward", "laya_n_act", "laya_max_len",
                 "laya_max_markers", "laya_temperature", "laya_prof_report", "laya_prof_reset", "laya_tune_all"]


def declared(header):
    src = open(os.path.join(REPO, "include", header)).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return re.findall(r"\b(laya_\w+)\s*\(", src)


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(le.DEFAULT_LIB):
        from layamd_amd import build
        build.build()
    return le.load_library()


def test_api_header_is_the_reference_abi():
    assert declared("laya_api.h") == REFERENCE_ABI


@pytest.mark.parametrize("header", ["laya_api.h", "laya_ext.h"])
def test_every_declared_symbol_is_exported(lib, header):
    names = declared(header)
    assert names
    for n in names:
        assert hasattr(lib, n), n


def test_binding_covers_the_headers():
    assert le.ABI_SYMBOLS == REFERENCE_ABI
    assert set(le.EXT_SYMBOLS) == set(declared("laya_ext.h"))


def test_product_library_does_not_link_the_oracle():
    data = open(le.DEFAULT_LIB, "rb").read()
    assert b"oracle" not in data and b"torch" not in data


@pytest.mark.parametrize("tool", ["laya-parity", "laya-bench"])
def test_cpp_tools_are_built_and_start_without_a_gpu(lib, tool):
    """The C++ callers of laya_api.h (built next to liblaya.so) link it and print their usage
    without touching a GPU when given no arguments."""
    import subprocess
    exe = os.path.join(os.path.dirname(le.DEFAULT_LIB), tool)
    assert os.path.exists(exe)
    r = subprocess.run([exe], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=60)
    assert r.returncode == 2 and "usage" in r.stdout


def _in_child(code):
    """Runs code in a fresh interpreter (a call the library should reject must not reach the HIP
    runtime, which has no device here; a wrong acceptance then ends only the child)."""
    import subprocess
    import sys
    r = subprocess.run([sys.executable, "-c", "import sys; sys.path.insert(0, %r)\n" % REPO + code],
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=120)
    return r.returncode, r.stdout


def test_hooks_reject_operands_beyond_32bit_offsets(lib):
    """laya_ext_gemm, laya_ext_gemm_splitk_static and laya_ext_attention refuse operands that the
    kernels' 32-bit buffer offsets cannot reach (GEMM: any operand of 4 GiB or more; attention: K or
    V^T of 2 GiB or more) before any HIP call, so no device is needed to see the -1."""
    rc, out = _in_child('''
import ctypes
from layamd_amd import engine as le
L = le.load_library()
P = ctypes.c_void_p(0x100000)          # aligned stand-ins: never dereferenced on the rejection path
# bf16 A of 2^20 rows x 2048 = 4 GiB
print(L.laya_ext_gemm(1, 0, P, P, P, None, 0, 1 << 20, 1024, 2048, None, 1, None))
# fp32 residual output of 2^20 x 1024 x 4 bytes = 4 GiB, with A below it
print(L.laya_ext_gemm(1, 1, P, P, P, None, 0, 1 << 20, 1024, 64, None, 1, None))
print(L.laya_ext_gemm_splitk_static(0, P, P, P, None, 0, 1 << 20, 1024, 2048, 2, None))
# attention: K of 2^20 rows x 1024 bf16 = 2 GiB
print(L.laya_ext_attention(1, P, P, 1024, 1 << 20, P, 4096, P, 1024, P, 1, 64, 16, P, P, None, None, 0,
                           ctypes.c_float(0.125), None))
# 128-query tiles with a window half width that is not a multiple of 64, and the gathered mode
# with a window: both refused instead of reaching the launcher
print(L.laya_ext_attention(1, P, P, 1024, 4096, P, 4224, P, 1024, P, 1, 128, 16, P, P, None, None, 32,
                           ctypes.c_float(0.125), None))
print(L.laya_ext_attention(1, P, P, 1024, 4096, P, 4224, P, 1024, P, 1, 64, 16, P, P, P, P, 64,
                           ctypes.c_float(0.125), None))
''')
    assert rc == 0, out
    assert out.split() == ["-1"] * 6, out


def test_parity_tool_fails_on_non_finite_outputs(lib):
    """laya-parity's comparison fails a question whose engine logits or act values hold NaN or +-Inf
    (a NaN difference must not read as 0), checked on planted values without an engine."""
    import subprocess
    exe = os.path.join(os.path.dirname(le.DEFAULT_LIB), "laya-parity")
    r = subprocess.run([exe, "--self-check"], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=60)
    assert r.returncode == 0 and "self-check: ok" in r.stdout, r.stdout


REF_SRC = "/root/reference/src"


@pytest.mark.skipif(not os.path.isdir(REF_SRC), reason="the reference sources are only in the build container")
@pytest.mark.parametrize("caller", ["test_parity.cpp", "bench_engine.cpp"])
def test_reference_callers_link_against_the_library(lib, caller, tmp_path):
    """The reference's own C++ callers of laya_api.h (src/test_parity.cpp, src/bench_engine.cpp)
    compile unchanged and link against liblaya.so; nothing is run.  A second translation unit
    includes both the reference's laya_api.h and include/laya_api.h, which the compiler accepts
    only if every shared declaration agrees."""
    import subprocess
    pkg = os.path.dirname(le.DEFAULT_LIB)
    exe = str(tmp_path / caller.replace(".cpp", ""))
    r = subprocess.run(["g++", "-std=c++17", "-O0", "-o", exe, os.path.join(REF_SRC, caller), "-L" + pkg, "-llaya",
                        "-Wl,-rpath," + pkg], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-3000:]
    both = tmp_path / "both.cpp"
    both.write_text('#include "%s/laya_api.h"\n#include "%s/include/laya_api.h"\nint main() { return 0; }\n'
                    % (REF_SRC, REPO))
    r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", str(both)], stdout=subprocess.PIPE,
                       stderr=subprocess.STDOUT, text=True, timeout=120)
    assert r.returncode == 0, r.stdout
