"""Clebsch-Gordan table of the reference, as data.

Restates: reference include/cg_coefficients_l3.cuh:19-831 (34 paths, 611
entries; path order l1 outer, l2, l_out inner -- python/cg_coefficients/
generate_cg.py:97-118) and src/tensor_product/tensor_product.cu:203-214
(get_num_paths_l3 / get_path_info_l3).  The numbers are loaded from
tests/golden/cg_l3_ref.json, which tests/golden/make_fixtures.py parsed out of
that header's text.
"""
import functools
import json
import os

import numpy as np

_FIXTURE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                        "tests", "golden", "cg_l3_ref.json")

NUM_PATHS = 34
NUM_ENTRIES = 611


@functools.lru_cache(maxsize=None)
def fixture():
    with open(_FIXTURE) as fh:
        return json.load(fh)


def path_info():
    """[34, 3] int32 (l1, l2, l_out) -- cg_coefficients_l3.cuh:796-831."""
    return np.array(fixture()["paths"], dtype=np.int32)


def entries():
    """[611, 5] float64: path, global a, global b, global o, coeff.

    Global component indices add the l^2 offsets of BLOCK_INFO
    (cg_coefficients_l3.cuh:23-58) to ENTRY_INFO's local indices (:99-711).
    """
    fx = fixture()
    out = []
    for p, m1, m2, mo, c in fx["entries"]:
        o1, o2, oo = fx["offsets"][p]
        out.append((p, o1 + m1, o2 + m2, oo + mo, c))
    return np.array(out, dtype=np.float64)


@functools.lru_cache(maxsize=None)
def dense():
    """Dense C[a, b, o] (16 x 16 x 16), summing all paths (they never overlap)."""
    c = np.zeros((16, 16, 16))
    for p, a, b, o, v in entries():
        c[int(a), int(b), int(o)] += v
    return c


@functools.lru_cache(maxsize=None)
def dense_paths():
    """Per-path blocks: C_p[a, b, q] with q the per-path output slot (156 slots).

    Slot q = sum_{p' < p} (2 l_out(p') + 1) + m_out -- the order in which the
    weighted product of tensor_product_fused.cuh:1509-2276 visits paths.
    """
    info = path_info()
    slots = np.concatenate([[0], np.cumsum(2 * info[:, 2] + 1)])
    c = np.zeros((16, 16, int(slots[-1])))
    fx = fixture()
    for p, m1, m2, mo, v in fx["entries"]:
        o1, o2, _ = fx["offsets"][p]
        c[o1 + m1, o2 + m2, slots[p] + mo] = v
    return c, slots


def slot_to_output():
    """[156] output component (0..15) of every per-path slot."""
    info = path_info()
    out = []
    for l1, l2, lo in info:
        out.extend(range(lo * lo, lo * lo + 2 * lo + 1))
    return np.array(out)


def slot_to_path():
    info = path_info()
    out = []
    for p, (_, _, lo) in enumerate(info):
        out.extend([p] * (2 * lo + 1))
    return np.array(out)
