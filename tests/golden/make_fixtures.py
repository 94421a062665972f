#!/usr/bin/env python3
"""Write the golden fixtures under tests/golden/ from the reference's data files.

The reference ships no golden-vector files.  Its only fixed data for this path
is the Clebsch-Gordan table vendored as text in
  /root/reference/include/cg_coefficients_l3.cuh
    BLOCK_INFO  :23-58   (l1, l2, l_out, offsets per path)
    BLOCK_RANGES:61-96   (entry range per path)
    ENTRY_INFO  :99-711  (m1, m2, m_out per entry)
    CG_COEFFS   :714-792 (fp32 coefficient per entry)
This script reads those arrays as numbers (no code is imported or run) and
stores them as JSON data: cg_l3_ref.json.

It also writes the known-answer spherical-harmonic inputs the reference tests
use (tests/test_spherical_harmonics.py:55-62 axis vectors, :76-82 diagonal
vectors, :94-99 near-pole vectors) as sh_known_inputs.json.  The expected
values for those inputs are fixed by hand-computable closed forms and are
asserted in tests/test_oracle_sh.py.

Run in the build container (where /root/reference exists):
    python tests/golden/make_fixtures.py
"""
import json
import os
import re

REF = "/root/reference/include/cg_coefficients_l3.cuh"
HERE = os.path.dirname(os.path.abspath(__file__))


def _array_text(txt, name):
    i = txt.index(name)
    j = txt.index("};", i)
    return txt[i:j]


def cg_fixture():
    txt = open(REF).read()
    info = [tuple(map(int, m)) for m in re.findall(
        r"\{(-?\d+), (-?\d+), (-?\d+), (-?\d+), (-?\d+), (-?\d+)\}",
        _array_text(txt, "BLOCK_INFO[NUM_BLOCKS][6]"))]
    ranges = [tuple(map(int, m)) for m in re.findall(
        r"\{(\d+), (\d+)\}", _array_text(txt, "BLOCK_RANGES[NUM_BLOCKS][2]"))]
    entries = [tuple(map(int, m)) for m in re.findall(
        r"\{(\d+), (\d+), (\d+)\}", _array_text(txt, "ENTRY_INFO[NUM_ENTRIES][3]"))]
    coeffs = [float(x) for x in re.findall(
        r"(-?\d+\.\d+)f", _array_text(txt, "CG_COEFFS[NUM_ENTRIES]"))]
    assert len(info) == 34 and len(ranges) == 34
    assert len(entries) == 611 and len(coeffs) == 611
    rows = []
    for p, (s, e) in enumerate(ranges):
        for k in range(s, e):
            rows.append([p, entries[k][0], entries[k][1], entries[k][2], coeffs[k]])
    return {
        "source": "reference include/cg_coefficients_l3.cuh:23-792 (values only)",
        "paths": [list(r[:3]) for r in info],
        "offsets": [list(r[3:]) for r in info],
        "entries": rows,  # [path, m1_idx, m2_idx, mout_idx, coeff]
    }


def sh_inputs():
    s2 = 1.0 / 2 ** 0.5
    s3 = 1.0 / 3 ** 0.5
    return {
        "source": "reference tests/test_spherical_harmonics.py:55-62,76-82,94-99",
        "axis": [[1, 0, 0], [-1, 0, 0], [0, 1, 0], [0, -1, 0], [0, 0, 1], [0, 0, -1]],
        "diagonal": [[s2, s2, 0], [s2, 0, s2], [0, s2, s2], [s3, s3, s3], [-s3, s3, s3]],
        "near_pole_unnormalised": [[1e-7, 0, 1], [0, 1e-7, 1], [1e-7, 1e-7, 1], [1e-7, 0, -1]],
    }


if __name__ == "__main__":
    with open(os.path.join(HERE, "cg_l3_ref.json"), "w") as fh:
        fx = cg_fixture()
        fh.write("{\n")
        fh.write('"source": %s,\n' % json.dumps(fx["source"]))
        fh.write('"paths": %s,\n' % json.dumps(fx["paths"]))
        fh.write('"offsets": %s,\n' % json.dumps(fx["offsets"]))
        fh.write('"entries": [\n' + ",\n".join(json.dumps(r) for r in fx["entries"]) + "\n]\n}\n")
    with open(os.path.join(HERE, "sh_known_inputs.json"), "w") as fh:
        json.dump(sh_inputs(), fh, indent=1)
    print("fixtures written to", HERE)
