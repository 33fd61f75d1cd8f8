"""Builds the native libraries of cppnet_amd in-tree.

  cppnet_amd/_lib/libcnhip.so    HIP kernels for gfx950 + the C ABI (include/cnhip.h)
  cppnet_amd/_lib/libcppnet.so   C++17 CppNet-compatible host layer + trainer C ABI
                                 (include/cppnet_train.h), linked to libcnhip.so

Usage: python -m cppnet_amd.build  (or cppnet_amd.build.build_all()).
Every call recompiles every source; objects are compiled in parallel.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
HOST = CSRC / "host"
LIBDIR = PKG / "_lib"
OBJDIR = PKG / "_build"
INCLUDE = ROOT / "include"
HOST_INCLUDE = PKG / "include"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Wno-unused-function",
    # Packed fp32 (v_pk_*_f32) code generation stays off for all device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
    f"-I{INCLUDE}", f"-I{CSRC}",
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", f"-I{INCLUDE}", f"-I{HOST_INCLUDE}"]


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in res.stdout.splitlines()
                    if "packed-fp32-ops" not in l and l.strip() != "1 warning generated.")
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def _jobs() -> int:
    try:
        return max(1, min(16, int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    except ValueError:
        return 4


def build_hip() -> Path:
    srcs = sorted(CSRC.glob("*.hip"))
    OBJDIR.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    objs = [OBJDIR / (s.stem + ".o") for s in srcs]
    with ThreadPoolExecutor(_jobs()) as ex:
        list(ex.map(lambda so: _run([HIPCC, *HIP_FLAGS, "-c", str(so[0]), "-o", str(so[1])]),
                    zip(srcs, objs)))
    out = LIBDIR / "libcnhip.so"
    tmp = LIBDIR / "libcnhip.so.tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, out)
    return out


def build_host() -> Path | None:
    srcs = sorted(HOST.glob("*.cpp"))
    if not srcs:
        return None
    objs = [OBJDIR / ("host_" + s.stem + ".o") for s in srcs]
    with ThreadPoolExecutor(_jobs()) as ex:
        list(ex.map(lambda so: _run([CXX, *CXX_FLAGS, "-c", str(so[0]), "-o", str(so[1])]),
                    zip(srcs, objs)))
    out = LIBDIR / "libcppnet.so"
    tmp = LIBDIR / "libcppnet.so.tmp"
    _run([CXX, "-shared", "-fPIC", "-o", str(tmp), *map(str, objs), f"-L{LIBDIR}", "-lcnhip",
          "-Wl,-rpath,$ORIGIN", "-Wl,--no-undefined"])
    os.replace(tmp, out)
    return out


def build_all() -> None:
    build_hip()
    build_host()
    shutil.rmtree(OBJDIR, ignore_errors=True)


if __name__ == "__main__":
    build_all()
    print("built", *sorted(p.name for p in LIBDIR.glob("*.so")))
