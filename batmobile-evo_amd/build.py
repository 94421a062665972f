#!/usr/bin/env python3
"""Build the batmobile MI355X library and its PyTorch extension, in-tree.

  lib/libbatmobile_hip.so         HIP kernels + C ABI (include/batmobile_hip.h),
                                  hipcc --offload-arch=gfx950
  lib/libbatteries_neighbor.so    the neighbor list alone (the reference's ctypes
                                  library name: neighbor_list_cuda / _free /
                                  _estimate_memory and the batteries_neighbor_list_*
                                  entry points), from the same object
  python/_batmobile.so            torch extension (host code only) over the C ABI

Usage:  python build.py [--force]
"""
import argparse
import concurrent.futures as cf
import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(REPO, "include")
BUILD = os.path.join(HERE, "_build")
LIBDIR = os.path.join(HERE, "lib")
PYDIR = os.path.join(HERE, "python")
LIB = os.path.join(LIBDIR, "libbatmobile_hip.so")
NL_LIB = os.path.join(LIBDIR, "libbatteries_neighbor.so")
EXT = os.path.join(PYDIR, "_batmobile" + sysconfig.get_config_var("EXT_SUFFIX"))

HIP_SOURCES = ["sh.hip", "tp.hip", "mp.hip", "nl.hip", "graph.hip", "mace.hip"]
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # packed FP32 (v_pk_*_f32) generation off; see the kernels' notes
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + CSRC, "-I" + INCLUDE,
]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError("command failed:\n  " + " ".join(cmd) + "\n" + out)
    return out


def _stale(target, deps):
    if not os.path.exists(target):
        return True
    t = os.path.getmtime(target)
    return any(os.path.getmtime(d) > t for d in deps)


def _headers():
    hs = [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")]
    hs += [os.path.join(INCLUDE, f) for f in os.listdir(INCLUDE) if f.endswith(".h")]
    return hs


def build_lib(force=False, jobs=4):
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    hdrs = _headers()
    objs, todo = [], []
    for src in HIP_SOURCES:
        s = os.path.join(CSRC, src)
        o = os.path.join(BUILD, src.replace(".hip", ".o"))
        objs.append(o)
        if force or _stale(o, [s] + hdrs):
            todo.append([HIPCC] + HIP_FLAGS + ["-c", s, "-o", o])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, todo))
    if force or todo or _stale(LIB, objs):
        _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", LIB] + objs)
    nl_obj = os.path.join(BUILD, "nl.o")
    if force or todo or _stale(NL_LIB, [nl_obj]):
        _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", NL_LIB, nl_obj])
    return LIB


def build_ext(force=False):
    import torch
    from torch.utils import cpp_extension

    src = os.path.join(CSRC, "binding.cpp")
    if not (force or _stale(EXT, [src, LIB] + _headers())):
        return EXT
    inc = cpp_extension.include_paths() + [os.path.join(ROCM, "include"), INCLUDE,
                                          sysconfig.get_paths()["include"]]
    torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", src, "-o", EXT,
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DTORCH_EXTENSION_NAME=_batmobile",
           "-DTORCH_API_INCLUDE_EXTENSION_H", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           "-w"]
    cmd += ["-I" + p for p in inc]
    cmd += ["-L" + torch_lib, "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
            "-L" + LIBDIR, "-lbatmobile_hip", "-L" + os.path.join(ROCM, "lib"), "-lamdhip64",
            "-Wl,-rpath,$ORIGIN/../lib", "-Wl,-rpath," + torch_lib]
    _run(cmd)
    return EXT


def build(force=False):
    build_lib(force=force)
    build_ext(force=force)
    return LIB, NL_LIB, EXT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--force", action="store_true")
    a = ap.parse_args()
    for p in build(force=a.force):
        print("built", p)
    sys.exit(0)
