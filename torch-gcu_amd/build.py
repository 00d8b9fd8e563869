"""Build script for the torch_gcu MI355X extension.

Two shared libraries are produced in-tree:

* ``torch_gcu/lib/libmi355x_ops.so`` -- the hand-written gfx950 HIP kernels
  behind the C ABI declared in ``include/mi355x_ops.h`` (no torch dependency).
* ``torch_gcu/_C.so`` -- the C++ host: the PrivateUse1 runtime (device guard,
  streams, caching allocator, GCUGraph), the generated operator
  registrations and the efficient ops, linked against the kernel library.

Every call compiles from scratch (objects go to ``_build/``).  Usage::

    python torch-gcu_amd/build.py [--kernels-only] [-j N]
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
INCLUDE = os.path.join(REPO, "include")
KERNEL_DIR = os.path.join(HERE, "csrc", "kernels")
HOST_DIR = os.path.join(HERE, "csrc", "host")
PKG = os.path.join(HERE, "torch_gcu")
LIB_DIR = os.path.join(PKG, "lib")
BUILD = os.path.join(HERE, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = os.environ.get("MI_OFFLOAD_ARCH", "gfx950")

KERNEL_LIB = os.path.join(LIB_DIR, "libmi355x_ops.so")
HOST_LIB = os.path.join(PKG, "_C" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so"))

# Packed fp32 instructions are kept out of every HIP object.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result", "-munsafe-fp-atomics",
]


INCREMENTAL = False  # development only: skip objects newer than their sources


def _up_to_date(src: str, obj: str, deps: list[str]) -> bool:
    if not INCREMENTAL or not os.path.exists(obj):
        return False
    t = os.path.getmtime(obj)
    return all(os.path.getmtime(d) < t for d in [src, *deps])


def _run(cmd: list[str], what: str) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(
        line for line in (proc.stdout + proc.stderr).splitlines()
        if "packed-fp32-ops" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({what}):\n{' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def _sources(d: str, exts: tuple[str, ...]) -> list[str]:
    return sorted(os.path.join(d, f) for f in os.listdir(d) if f.endswith(exts))


def build_kernels(jobs: int) -> str:
    os.makedirs(os.path.join(BUILD, "kernels"), exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    srcs = _sources(KERNEL_DIR, (".hip", ".cpp"))
    objs = []
    cmds = []
    for s in srcs:
        o = os.path.join(BUILD, "kernels", os.path.basename(s) + ".o")
        objs.append(o)
        lang = ["-x", "hip"] if s.endswith(".hip") else []
        if _up_to_date(s, o, _sources(KERNEL_DIR, (".h",)) + [os.path.join(INCLUDE, "mi355x_ops.h")]):
            continue
        cmds.append(([HIPCC, *HIP_FLAGS, *lang, "-I", INCLUDE, "-I", KERNEL_DIR, "-c", s, "-o", o],
                     os.path.basename(s)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda c: _run(*c), cmds))
    tmp = KERNEL_LIB + ".tmp"
    _run([HIPCC, *HIP_FLAGS, "-shared", "-o", tmp, *objs,
          "-Wl,-soname,libmi355x_ops.so"], "link kernels")
    os.replace(tmp, KERNEL_LIB)
    return KERNEL_LIB


def _torch_flags() -> tuple[list[str], list[str]]:
    import torch
    from torch.utils import cpp_extension

    inc = [f"-I{p}" for p in cpp_extension.include_paths()]
    inc += [f"-I{sysconfig.get_paths()['include']}", f"-I{ROCM}/include"]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cflags = ["-O2", "-fPIC", "-std=c++17", "-D__HIP_PLATFORM_AMD__=1",
              f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DTORCH_EXTENSION_NAME=_C",
              "-DTORCH_API_INCLUDE_EXTENSION_H", "-Wno-deprecated-declarations",
              "-fvisibility=hidden"]
    torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    ldflags = [f"-L{torch_lib}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python",
               f"-L{LIB_DIR}", "-lmi355x_ops", f"-L{torch_lib}", "-lamdhip64",
               "-Wl,-rpath,$ORIGIN/lib", f"-Wl,-rpath,{torch_lib}"]
    return inc + cflags, ldflags


def build_host(jobs: int) -> str:
    gen_dir = os.path.join(BUILD, "generated")
    os.makedirs(gen_dir, exist_ok=True)
    sys.path.insert(0, os.path.join(HERE, "codegen"))
    import gen_register  # noqa: E402

    generated = gen_register.generate(gen_dir)
    cflags, ldflags = _torch_flags()
    srcs = _sources(HOST_DIR, (".cpp",)) + generated
    os.makedirs(os.path.join(BUILD, "host"), exist_ok=True)
    objs, cmds = [], []
    for s in srcs:
        o = os.path.join(BUILD, "host", os.path.basename(s) + ".o")
        objs.append(o)
        if _up_to_date(s, o, _sources(HOST_DIR, (".h",)) + [os.path.join(gen_dir, "aotops.h")]):
            continue
        cmds.append((["g++", *cflags, "-I", INCLUDE, "-I", HOST_DIR, "-I", gen_dir, "-c", s,
                      "-o", o], os.path.basename(s)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda c: _run(*c), cmds))
    tmp = HOST_LIB + ".tmp"
    _run(["g++", "-shared", "-o", tmp, *objs, *ldflags], "link host")
    os.replace(tmp, HOST_LIB)
    return HOST_LIB


def build(kernels_only: bool = False, jobs: int | None = None) -> None:
    jobs = jobs or min(8, os.cpu_count() or 4)
    if os.path.isdir(BUILD) and not INCREMENTAL:
        shutil.rmtree(BUILD)
    build_kernels(jobs)
    if not kernels_only and os.path.isdir(HOST_DIR) and _sources(HOST_DIR, (".cpp",)):
        build_host(jobs)


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--kernels-only", action="store_true")
    ap.add_argument("-j", type=int, default=None)
    ap.add_argument("--incremental", action="store_true",
                    help="development: reuse objects newer than their sources")
    a = ap.parse_args()
    INCREMENTAL = a.incremental
    build(a.kernels_only, a.j)
    print("built", KERNEL_LIB, "" if a.kernels_only else HOST_LIB)
