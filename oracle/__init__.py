"""CPU oracle for the batmobile equivariant message-passing path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library, the
`_batmobile` extension, the `batmobile` package) may import, call, link or
execute anything under oracle/.  Only tests/, __graft_entry__.smoke() and the
`cpu_baseline` leg of bench.py use it, and only as the checker.

Every function restates the reference's algorithm in float64 numpy (or plain C
for the neighbor list, oracle/nl_ref.c) and cites the reference file:line it
follows.  How each function is pinned:

  cg       reference table values (tests/golden/cg_l3_ref.json, parsed from
           include/cg_coefficients_l3.cuh) + orthonormality + exact +-sqrt(p/q)
           + intertwiner property w.r.t. the SH basis + product rule.
  sh       closed-form known answers (axis vectors), component normalisation
           sum_m Y_lm^2 = 2l+1, CG product rule Y_{l+1} ~ CG(Y_l, r),
           harmonicity, rotation equivariance.
  sh_grad  central finite differences; torch.autograd of the forward.
  tp_*     brute-force loops on tiny inputs, equivariance, adjoint identity
           <TP(x,y), g> = <x, gx> = <y, gy>, finite differences.
  mp_*     composition identities (fused == SH->TP->index_add), per-edge loop.
  nl       brute force over all pairs (same fp32 op order), symmetry,
           hand-made lattice known answers.
  mace     (the per-edge-weight layer of configs[4], defined here: no reference
           API has per-edge weights) envelope values and vanishing derivatives,
           Bessel orthonormality, unit weights reducing to TP_simple, finite
           differences and translation invariance of the position gradient.
"""
