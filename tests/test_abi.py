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
