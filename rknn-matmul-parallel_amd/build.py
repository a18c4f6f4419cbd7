"""Build the MI355X decoder library in-tree.

Produces, next to this file:
  lib/libmatmul_decoder.so   the C ABI (matmul_decoder.h, rknn_matmul_parallel.h,
                             mdx_ext.h): host C runtime + gfx950 HIP kernels
  matmul_decoder<ext>.so     the pybind11 module with the reference's Python surface

Kernels: hipcc --offload-arch=gfx950 -O3, packed-fp32 instructions disabled,
no floating-point contraction (every a*b+c rounds twice unless a fused builtin
is written).  Host C: gcc -O2 -std=c11.  Run `python build.py` or call build().
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
INC = os.path.join(ROOT, "include")
KDIR = os.path.join(HERE, "csrc", "kernels")
HDIR = os.path.join(HERE, "csrc", "host")
PDIR = os.path.join(HERE, "csrc", "pybind")
BUILD = os.path.join(HERE, "_build")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libmatmul_decoder.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

HIP_FLAGS = [
    "-O3", "-fPIC", "-std=c++17", f"--offload-arch={ARCH}", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-I", INC, "-I", KDIR,
]
C_FLAGS = ["-O2", "-fPIC", "-std=gnu11", "-Wall", "-Wextra", "-Wno-unused-parameter",
           "-Wno-format-truncation", "-ffp-contract=off", "-I", INC, "-I", KDIR, "-I", HDIR]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def _sources(d: str, ext: str) -> list[str]:
    return sorted(os.path.join(d, f) for f in os.listdir(d) if f.endswith(ext))


def _obj(src: str) -> str:
    return os.path.join(BUILD, os.path.basename(src) + ".o")


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile every kernel and host source and link the library and module."""
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    cmds = []
    for s in _sources(KDIR, ".hip"):
        cmds.append([HIPCC, *HIP_FLAGS, "-c", s, "-o", _obj(s)])
    for s in _sources(HDIR, ".c"):
        cmds.append(["gcc", *C_FLAGS, "-c", s, "-o", _obj(s)])
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for f in [ex.submit(_run, c) for c in cmds]:
            f.result()
    objs = [c[-1] for c in cmds]
    tmp = LIB + ".tmp"
    _run([HIPCC, "-shared", f"--offload-arch={ARCH}", "-o", tmp, *objs, "-lpthread", "-lm",
          "-Wl,-soname,libmatmul_decoder.so"])
    os.replace(tmp, LIB)
    # pybind11 module
    import pybind11
    ext = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    mod = os.path.join(HERE, "matmul_decoder" + ext)
    py_inc = sysconfig.get_paths()["include"]
    _run(["g++", "-O2", "-shared", "-fPIC", "-std=c++17", "-I", INC, "-I", py_inc,
          "-I", pybind11.get_include(), os.path.join(PDIR, "matmul_decoder_py.cpp"),
          "-L", LIBDIR, "-lmatmul_decoder", "-Wl,-rpath,$ORIGIN/lib", "-o", mod + ".tmp"])
    os.replace(mod + ".tmp", mod)
    if verbose:
        print(f"built {LIB}\nbuilt {mod}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
