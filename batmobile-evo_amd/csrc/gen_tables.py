#!/usr/bin/env python3
"""Generate the compile-time tables the HIP kernels are built on.

Everything here is derived from mathematics, not read from any other code:

* Real Clebsch-Gordan coefficients for l1, l2, l_out <= 3.  Complex (SU(2))
  coefficients come from the Racah formula; they are moved to the real
  spherical-harmonic basis with the unitary real->complex change of basis that
  carries an extra (-i)^l phase (this makes every coefficient real), and each
  (l1, l2, l_out) block is scaled to Frobenius norm sqrt(2*l_out+1)
  ("component" normalisation: cg = sqrt(2 l_out + 1) * wigner_3j).
  The path order (l1 outer, l2, l_out inner) and the entry order inside a path
  (m1, m2, m_out) are the ones the reference table uses
  (reference: python/cg_coefficients/generate_cg.py:97-118,
  include/cg_coefficients_l3.cuh:23-792); the test-suite checks every one of
  the 611 values against that table.

* Real spherical harmonics up to l = 6 as the recurrence
      Y_{l+1}[M] = k_l * sum_{m,j} CG(l,1,l+1)[m, j, M] * Y_l[m] * r_j ,
  r = (x, y, z) in the e3nn axis order (y is the polar axis), with the
  positive constant k_l fixed by sum_M Y_{l+1}[M]^2 = 2l+3 on the unit sphere.
  For l <= 3 this reproduces the closed-form polynomials of
  reference src/spherical_harmonics/spherical_harmonics.cu:56-96 and for
  l = 4..6 the coefficients of :99-256 (checked in the tests).

Run:  python gen_tables.py  -> writes generated_tables.h next to this file.
"""
import os
from math import factorial, sqrt

import numpy as np

LMAX_TP = 3
LMAX_SH = 6


def _su2_cg(j1, m1, j2, m2, j, m):
    """<j1 m1 j2 m2 | j m> by the Racah formula (integer spins only)."""
    if m1 + m2 != m or not abs(j1 - j2) <= j <= j1 + j2:
        return 0.0
    f = factorial
    pre = sqrt((2 * j + 1) * f(j + j1 - j2) * f(j - j1 + j2) * f(j1 + j2 - j)
               / f(j1 + j2 + j + 1))
    pre *= sqrt(f(j + m) * f(j - m) * f(j1 - m1) * f(j1 + m1) * f(j2 - m2) * f(j2 + m2))
    s = 0.0
    for k in range(0, j1 + j2 + j + 1):
        d = [k, j1 + j2 - j - k, j1 - m1 - k, j2 + m2 - k, j - j2 + m1 + k, j - j1 - m2 + k]
        if min(d) < 0:
            continue
        den = 1
        for v in d:
            den *= f(v)
        s += (-1) ** k / den
    return pre * s


def _real_to_complex(l):
    """Unitary Q with complex_Y = Q @ real_Y, including the (-i)^l phase."""
    q = np.zeros((2 * l + 1, 2 * l + 1), dtype=complex)
    r2 = 1.0 / sqrt(2.0)
    for m in range(-l, 0):
        q[l + m, l - m] = r2
        q[l + m, l + m] = -1j * r2
    q[l, l] = 1.0
    for m in range(1, l + 1):
        q[l + m, l + m] = (-1) ** m * r2
        q[l + m, l - m] = 1j * (-1) ** m * r2
    return (-1j) ** l * q


def real_cg(l1, l2, l3):
    """[2l1+1, 2l2+1, 2l3+1] real CG block with Frobenius norm sqrt(2l3+1)."""
    c = np.zeros((2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1))
    for m1 in range(-l1, l1 + 1):
        for m2 in range(-l2, l2 + 1):
            for m3 in range(-l3, l3 + 1):
                c[l1 + m1, l2 + m2, l3 + m3] = _su2_cg(l1, m1, l2, m2, l3, m3)
    q1, q2, q3 = _real_to_complex(l1), _real_to_complex(l2), _real_to_complex(l3)
    r = np.einsum("ij,kl,mn,ikn->jlm", q1, q2, np.conj(q3.T), c)
    assert np.abs(r.imag).max() < 1e-12
    r = r.real
    return r / np.linalg.norm(r) * sqrt(2 * l3 + 1)


def tp_paths(lmax=LMAX_TP):
    return [(l1, l2, l3) for l1 in range(lmax + 1) for l2 in range(lmax + 1)
            for l3 in range(lmax + 1) if abs(l1 - l2) <= l3 <= l1 + l2]


def tp_entries():
    """List of (path, m1_idx, m2_idx, mout_idx, coeff) in reference entry order."""
    out = []
    for p, (l1, l2, l3) in enumerate(tp_paths()):
        blk = real_cg(l1, l2, l3)
        for i in range(2 * l1 + 1):
            for j in range(2 * l2 + 1):
                for k in range(2 * l3 + 1):
                    if abs(blk[i, j, k]) > 1e-10:
                        out.append((p, i, j, k, float(blk[i, j, k])))
    return out


def sh_recurrence():
    """Per degree l+1 (1..LMAX_SH): list of (M, m, j, coeff) terms."""
    rng = np.random.default_rng(12345)
    u = rng.normal(size=3)
    u /= np.linalg.norm(u)
    y = [np.array([1.0])]
    steps = []
    for l in range(LMAX_SH):
        blk = real_cg(l, 1, l + 1)
        raw = np.einsum("mjM,m,j->M", blk, y[-1], u)
        k = sqrt((2 * l + 3) / float(np.sum(raw ** 2)))
        y.append(raw * k)
        terms = []
        for M in range(2 * l + 3):
            for m in range(2 * l + 1):
                for j in range(3):
                    v = blk[m, j, M] * k
                    if abs(v) > 1e-12:
                        terms.append((M, m, j, float(v)))
        steps.append(terms)
    return steps


def sh_polynomials(lmax=LMAX_TP):
    """The recurrence expanded into monomials: per degree l and component M a
    dict {(a, b, c): coeff} of x^a y^b z^c (homogeneous of degree l)."""
    steps = sh_recurrence()
    polys = [[{(0, 0, 0): 1.0}]]
    for l in range(lmax):
        new = [dict() for _ in range(2 * l + 3)]
        for (M, m, j, c) in steps[l]:
            for mono, v in polys[-1][m].items():
                e = list(mono)
                e[j] += 1
                e = tuple(e)
                new[M][e] = new[M].get(e, 0.0) + c * v
        polys.append([{k: v for k, v in d.items() if abs(v) > 1e-12} for d in new])
    return polys


def _flit(v):
    return repr(float(v)) + "f" if "e" in repr(float(v)) or "." in repr(float(v)) else repr(float(v)) + ".0f"


def render():
    paths = tp_paths()
    ents = tp_entries()
    lines = []
    w = lines.append
    w("// Generated by gen_tables.py -- do not edit by hand.")
    w("// Real Clebsch-Gordan table (L<=3, 34 paths, 611 entries) and the real")
    w("// spherical-harmonic recurrence (L<=6), both derived from first principles.")
    w("#pragma once")
    w("#include <cstdint>")
    w("")
    w("namespace bmhip {")
    w("")
    w(f"constexpr int kNumPaths = {len(paths)};")
    w(f"constexpr int kNumEntries = {len(ents)};")
    w("constexpr int kIrreps = 16;  // (3+1)^2 components for L_max = 3")
    w("")
    w("// (l1, l2, l_out) of each path, reference path order.")
    w("constexpr int kPathL[kNumPaths][3] = {")
    w(",\n".join(f"    {{{a}, {b}, {c}}}" for a, b, c in paths))
    w("};")
    w("")
    # per-path output slots: q = kPathSlot[p] + m_out, 156 in total
    slots, acc = [], 0
    for (_, _, l3) in paths:
        slots.append(acc)
        acc += 2 * l3 + 1
    w(f"constexpr int kNumSlots = {acc};  // sum over paths of (2 l_out + 1)")
    w("constexpr int kPathSlot[kNumPaths] = {" + ", ".join(map(str, slots)) + "};")
    slot_path = [p for p, (_, _, l3) in enumerate(paths) for _ in range(2 * l3 + 1)]
    slot_out = [l3 * l3 + m for (_, _, l3) in paths for m in range(2 * l3 + 1)]
    w("// path and output component (0..15) of every per-path slot")
    w("constexpr int kSlotPath[kNumSlots] = {" + ", ".join(map(str, slot_path)) + "};")
    w("constexpr int kSlotOut[kNumSlots] = {" + ", ".join(map(str, slot_out)) + "};")
    w("")
    w("struct CGEntry {")
    w("    int p;     // path")
    w("    int a;     // component of input1 (0..15)")
    w("    int b;     // component of input2 (0..15)")
    w("    int o;     // component of the output (0..15)")
    w("    int q;     // per-path output slot (0..kNumSlots-1)")
    w("    float c;   // coefficient")
    w("};")
    w("")
    # entries are grouped by path: path p owns kCG[kPathEntry[p] .. kPathEntry[p + 1])
    assert [e[0] for e in ents] == sorted(e[0] for e in ents)
    starts = [0]
    for p in range(len(paths)):
        starts.append(starts[-1] + sum(1 for e in ents if e[0] == p))
    w("constexpr int kPathEntry[kNumPaths + 1] = {" + ", ".join(map(str, starts)) + "};")
    w("")
    w("constexpr CGEntry kCG[kNumEntries] = {")
    rows = []
    for (p, i, j, k, c) in ents:
        l1, l2, l3 = paths[p]
        rows.append(f"    {{{p}, {l1*l1+i}, {l2*l2+j}, {l3*l3+k}, {slots[p]+k}, {_flit(c)}}}")
    w(",\n".join(rows))
    w("};")
    w("")
    steps = sh_recurrence()
    w("// Spherical-harmonic recurrence: Y_{l+1}[M] += c * Y_l[m] * r[j], r = (x, y, z).")
    w("struct SHTerm {")
    w("    int M;")
    w("    int m;")
    w("    int j;")
    w("    float c;")
    w("};")
    counts = [len(t) for t in steps]
    w("constexpr int kSHTermCount[" + str(LMAX_SH) + "] = {" + ", ".join(map(str, counts)) + "};")
    w("constexpr int kSHTermStart[" + str(LMAX_SH + 1) + "] = {"
      + ", ".join(str(sum(counts[:i])) for i in range(LMAX_SH + 1)) + "};")
    w(f"constexpr SHTerm kSHTerms[{sum(counts)}] = {{")
    rows = []
    for l, terms in enumerate(steps):
        for (M, m, j, c) in terms:
            rows.append(f"    {{{M}, {m}, {j}, {_flit(c)}}}  /* l={l+1} */")
    w(",\n".join(rows))
    w("};")
    w("")
    polys = sh_polynomials()
    w("// The recurrence expanded for L <= 3: Y[l*l + M] = sum coeff * x^a y^b z^c.")
    w("struct SHMono {")
    w("    int k;     // component 0..15")
    w("    int a, b, c;")
    w("    float v;")
    w("};")
    mono = [(l * l + M, e, v) for l in range(LMAX_TP + 1) for M, d in enumerate(polys[l])
            for e, v in sorted(d.items())]
    w(f"constexpr int kSHMonoCount = {len(mono)};")
    w("constexpr SHMono kSHMono[kSHMonoCount] = {")
    w(",\n".join(f"    {{{k}, {e[0]}, {e[1]}, {e[2]}, {_flit(v)}}}" for k, e, v in mono))
    w("};")
    w("")
    w("}  // namespace bmhip")
    w("")
    return "\n".join(lines)


if __name__ == "__main__":
    here = os.path.dirname(os.path.abspath(__file__))
    path = os.path.join(here, "generated_tables.h")
    with open(path, "w") as fh:
        fh.write(render())
    print("wrote", path)
