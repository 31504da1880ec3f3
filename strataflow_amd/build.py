"""Builds libsfa.so (the gfx950 HIP library) and the CPU oracle in-tree.

``python -m strataflow_amd.build`` compiles every ``csrc/*.hip`` with hipcc for
gfx950 only and links ``strataflow_amd/libsfa.so`` (the attention library);
``host/`` (the C++ page manager over it) becomes ``strataflow_amd/libsfa_host.so``;
it also builds ``oracle/liboracle.so`` (the CPU oracle the tests compare against) with make.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
HOST = PKG / "host"
OBJ = ROOT / "_build" / "obj"
LIB = PKG / "libsfa.so"
HOST_LIB = PKG / "libsfa_host.so"
ORACLE_DIR = ROOT / "oracle"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# Packed FP32 VALU ops are disabled for all device code (they have produced
# silent wrong results on this hardware); the host pass ignores the flag.
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def _run(cmd: list[str], cwd: Path | None = None) -> None:
    proc = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def build_hip(verbose: bool = False) -> Path:
    OBJ.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")

    def compile_one(src: Path) -> Path:
        obj = OBJ / (src.stem + ".o")
        cmd = [HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), file=sys.stderr)
        _run(cmd)
        return obj

    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(compile_one, sources))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    return LIB


def build_host(verbose: bool = False) -> Path:
    """The host page manager: plain C++ with g++, the HIP part with hipcc,
    linked against libsfa.so (found next to it at run time)."""
    OBJ.mkdir(parents=True, exist_ok=True)
    objs = []
    for src in sorted(HOST.glob("*.cpp")):
        obj = OBJ / ("host_" + src.stem + ".o")
        cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-Wall", f"-I{HOST}", "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), file=sys.stderr)
        _run(cmd)
        objs.append(obj)
    for src in sorted(HOST.glob("*.hip")):
        obj = OBJ / ("host_" + src.stem + ".o")
        cmd = [HIPCC, *HIP_FLAGS, f"-I{HOST}", "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), file=sys.stderr)
        _run(cmd)
        objs.append(obj)
    tmp = HOST_LIB.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs),
          f"-L{PKG}", "-lsfa", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, HOST_LIB)
    return HOST_LIB


def build_oracle() -> Path:
    make = shutil.which("make")
    if make is None:
        raise RuntimeError("make not found")
    _run([make, "-s", "-B", "-C", str(ORACLE_DIR)])
    return ORACLE_DIR / "liboracle.so"


def build_all(verbose: bool = False) -> None:
    build_hip(verbose)
    build_host(verbose)
    build_oracle()


if __name__ == "__main__":
    build_all(verbose="-v" in sys.argv)
    print(f"built {LIB}")
