"""CPU tests of the host page manager: the C++ bookkeeping unit test and the
C ABI of libsfa_host.so (symbols only; no device calls without a GPU)."""
import ctypes
import subprocess
from pathlib import Path

import pytest

from strataflow_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HOST = ROOT / "strataflow_amd" / "host"


def test_page_planner_cpp(tmp_path):
    exe = tmp_path / "page_planner_test"
    subprocess.run(["g++", "-O1", "-std=c++17", "-Wall", "-Werror", f"-I{HOST}",
                    str(ROOT / "tests" / "cpp" / "page_planner_test.cpp"),
                    str(HOST / "page_planner.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    assert out.startswith("ok ")
    assert int(out.split()[1]) > 1000


def test_host_lib_exports():
    lib = _lib.load_host()
    for name in _lib.HOST_EXPORTS:
        assert hasattr(lib, name), name
    header = (ROOT / "include" / "sfa_pager.h").read_text()
    declared = {line.split("(")[0].split()[-1].lstrip("*")
                for line in header.splitlines() if line.startswith("SFA_API")}
    assert declared == set(_lib.HOST_EXPORTS)


def test_pager_config_layout():
    # the ctypes mirror of sfa_pager_config: 12 int32 then a uint64
    assert ctypes.sizeof(_lib.SfaPagerConfig) == 12 * 4 + 8
    assert _lib.SfaPagerConfig.seed.offset == 48
    assert ctypes.sizeof(_lib.SfaPagerStats) == 7 * 8


def test_pager_rejects_bad_config():
    lib = _lib.load_host()
    h = ctypes.c_void_p()
    bad = _lib.SfaPagerConfig(0, 32, 8, 128, 1, 256, 1, 4096, 0, 0, 0, 0, 0)  # n_layer 0
    assert lib.sfa_pager_create(ctypes.byref(bad), ctypes.byref(h)) == _lib.SFA_ERR_INVALID_ARGUMENT
    bad = _lib.SfaPagerConfig(1, 32, 8, 128, 1, 256, 1, 4096, 0, 7, 0, 0, 0)  # attend mode 7
    assert lib.sfa_pager_create(ctypes.byref(bad), ctypes.byref(h)) == _lib.SFA_ERR_INVALID_ARGUMENT
    bad = _lib.SfaPagerConfig(1, 32, 8, 96, 1, 256, 1, 4096, 0, 0, 0, 0, 0)  # head_dim 96
    assert lib.sfa_pager_create(ctypes.byref(bad), ctypes.byref(h)) != _lib.SFA_OK
    assert not h.value
    assert lib.sfa_pager_begin(None, None, None) == _lib.SFA_ERR_INVALID_ARGUMENT


def test_pager_valid_config_reaches_allocation():
    # a valid configuration passes validation; without a GPU the first device
    # allocation fails (out of memory or runtime error), never invalid argument
    import torch
    if torch.cuda.is_available():
        pytest.skip("CPU-only check")
    lib = _lib.load_host()
    h = ctypes.c_void_p()
    ok = _lib.SfaPagerConfig(2, 32, 8, 128, 1, 256, 4, 8192, 1024, 0, 0, 0, 1)
    rc = lib.sfa_pager_create(ctypes.byref(ok), ctypes.byref(h))
    assert rc in (_lib.SFA_ERR_OUT_OF_MEMORY, _lib.SFA_ERR_RUNTIME), rc
    assert not h.value
