"""The C ABI from a C99 program: include/sfa.h and include/sfa_pager.h compile
as C, the program links against libsfa.so and libsfa_host.so, and host-only
entry points behave as documented (no GPU needed)."""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_c_program_links_and_runs(tmp_path):
    lib_dir = ROOT / "strataflow_amd"
    exe = tmp_path / "c_abi_test"
    cmd = ["gcc", "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror", f"-I{ROOT / 'include'}",
           str(ROOT / "tests" / "cpp" / "c_abi_test.c"), "-o", str(exe), f"-L{lib_dir}", "-lsfa_host", "-lsfa",
           f"-Wl,-rpath,{lib_dir}"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    assert "c abi ok" in r.stdout
