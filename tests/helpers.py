"""Shared helpers of the test suite: seeded inputs, tensor layouts, tolerances."""
import numpy as np

from einsum_ir_amd import binary_loops

# tolerances stated by the task: relative Frobenius error
TOL_FP32 = 1e-5
TOL_BF16 = 2e-3
# fp64: no bar is stated for it; fp64 accumulation against the oracle's fp64
# accumulation differs only by summation order (~1e-16 * sqrt(K) relative)
TOL_FP64 = 1e-12


def uniform(rng, n, dtype=np.float32):
    """i.i.d. uniform[-1, 1]."""
    return rng.uniform(-1.0, 1.0, size=n).astype(dtype)


def rel_frobenius(ref, x):
    """||ref - x||_F / ||ref||_F in double precision (complex arrays compared
    as complex: both the real and the imaginary parts count)."""
    cpx = np.iscomplexobj(ref) or np.iscomplexobj(x)
    ref = np.asarray(ref, dtype=np.complex128 if cpx else np.float64).ravel()
    x = np.asarray(x, dtype=np.complex128 if cpx else np.float64).ravel()
    nrm = np.linalg.norm(ref)
    if nrm == 0.0:
        return float(np.linalg.norm(x))
    return float(np.linalg.norm(ref - x) / nrm)


def tensor_numel(dims, sizes):
    n = 1
    for d in dims:
        n *= sizes[d]
    return n


def parse_binary(expr):
    expr = expr.replace(" ", "")
    lhs, out = expr.split("->")
    left, right = lhs.split(",")
    return left, right, out


def loops_for(expr, sizes, **outer):
    return binary_loops(expr, sizes, **outer)
