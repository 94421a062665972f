"""ctypes wrapper around oracle/nl_ref.c (built into oracle/_build/libnl_ref.so).

TEST INFRASTRUCTURE ONLY.  See nl_ref.c for the reference lines restated.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "libnl_ref.so")


def build(force=False):
    if os.path.exists(LIB) and not force:
        return LIB
    os.makedirs(os.path.dirname(LIB), exist_ok=True)
    subprocess.check_call(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-fPIC",
                           "-shared", "-o", LIB, os.path.join(HERE, "nl_ref.c"), "-lm"])
    return LIB


_lib = None


def _load():
    global _lib
    if _lib is None:
        _lib = ctypes.CDLL(build())
        for name in ("nl_cell_list", "nl_brute_force"):
            f = getattr(_lib, name)
            f.restype = ctypes.c_int64
            f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_float,
                          ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                          ctypes.c_void_p]
    return _lib


def _run(name, pos, cell, cutoff, self_loops):
    pos = np.ascontiguousarray(pos, dtype=np.float32)
    cell = np.ascontiguousarray(cell, dtype=np.float32).reshape(9)
    n = pos.shape[0]
    f = getattr(_load(), name)
    cap = max(1024, 64 * n)
    while True:
        src = np.empty(cap, np.int32)
        dst = np.empty(cap, np.int32)
        vec = np.empty((cap, 3), np.float32)
        e = f(pos.ctypes.data, cell.ctypes.data, n, ctypes.c_float(cutoff), int(self_loops),
              cap, src.ctypes.data, dst.ctypes.data, vec.ctypes.data)
        if e <= cap:
            break
        cap = int(e)
    src, dst, vec = src[:e], dst[:e], vec[:e]
    order = np.lexsort((dst, src))
    return src[order], dst[order], vec[order]


def cell_list(pos, cell, cutoff, self_loops=False):
    """(src, dst, vec) sorted by (src, dst); vec = minimum-image pos[dst] - pos[src]."""
    return _run("nl_cell_list", pos, cell, cutoff, self_loops)


def brute_force(pos, cell, cutoff, self_loops=False):
    return _run("nl_brute_force", pos, cell, cutoff, self_loops)
