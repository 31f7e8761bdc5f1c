"""Builds the in-tree HIP library wisp_amd/libwisp_amd.so for gfx950.

Plain hipcc invocations (no CMake): each source in wisp_amd/csrc is compiled
to an object under wisp_amd/_build/ in parallel, then linked into one shared
library next to this file. Run: python -m wisp_amd.build
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "libwisp_amd.so"
INCLUDE = HERE.parent / "include"

ARCH = os.environ.get("WISP_AMD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: keep the compiler from forming v_pk_{add,mul,fma}_f32.
HIP_FLAGS = [
    "-O3", "-fPIC", "-std=c++17", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    f"-I{INCLUDE}",
]
HOST_CXX_FLAGS = ["-O2", "-fPIC", "-std=c++17", "-Wall", "-D__HIP_PLATFORM_AMD__",
                  f"-I{INCLUDE}", "-I/opt/rocm/include"]
HOST_C_FLAGS = ["-O2", "-fPIC", "-std=gnu11", "-Wall", "-Wextra", "-Wno-unused-parameter",
                "-D__HIP_PLATFORM_AMD__", f"-I{INCLUDE}", "-I/opt/rocm/include", "-pthread"]


def _sources():
    hip = sorted(CSRC.glob("*.hip"))
    cpp = sorted(CSRC.glob("*.cpp"))
    c = sorted(CSRC.glob("*.c"))
    return hip, cpp, c


def _compile(src: Path) -> Path:
    obj = BUILD / (src.name + ".o")
    if src.suffix == ".hip":
        cmd = [HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    elif src.suffix == ".cpp":
        cmd = ["g++", *HOST_CXX_FLAGS, "-c", str(src), "-o", str(obj)]
    else:
        cmd = ["gcc", *HOST_C_FLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    warn = [ln for ln in r.stderr.splitlines()
            if "warning" in ln and "packed-fp32-ops" not in ln]
    if warn:
        sys.stderr.write("\n".join(warn) + "\n")
    return obj


def build(verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    hip, cpp, c = _sources()
    srcs = hip + cpp + c
    jobs = min(len(srcs), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", f"--offload-arch={ARCH}", "-fPIC", "-o", str(tmp),
           *map(str, objs), "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    return LIB


if __name__ == "__main__":
    build()
