"""CPU oracle for the GLA hot path -- TEST INFRASTRUCTURE ONLY.

This package is a float64 NumPy restatement of the reference's `tops/cpu`
golden tier (the pure-JAX CPU reference of Fred33146/pallas-kernel).  It is
the checker the HIP kernels are compared against; it is never shipped or
measured as the product.  Only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may import it.

Every function cites the reference file:line it restates.  All arithmetic is
float64 ("fp64 mode" of tops/cpu, where every precision cast is a no-op), so
the oracle is evaluated on exactly the (bf16- or fp32-valued) inputs the
kernel saw, promoted to float64.

Pinning (see tests/test_oracle_*.py): each function is checked against an
independent formulation -- the per-token naive recurrence, the quadratic
"parallel form" with an explicit decay mask, torch float64 autograd of that
parallel form for every gradient, textbook causal linear attention for the
zero-gate case, and structural invariants (varlen == independent sequences,
state split == full run, g_gamma == broadcast g).
"""
