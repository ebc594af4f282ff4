"""GPU parity of complex contractions (CPX_MADD) and complex einsum
expressions.

The reference runs complex kernels on its BLAS backend
(reference src/backend/BinaryContractionBlas.cpp:68-85) and builds complex
trees in EinsumExpression (src/frontend/EinsumExpression.cpp:214-330, tests
EinsumExpression.test.torch.cpp:100-205 "batch-outer" / "batch-inner complex
matmul").  Here one loop of the IR is the complex dim (size 2, its stride
locating the imaginary parts) and the HIP kernels compute
out = sum_k A*B in complex arithmetic.  Checker: numpy.einsum in complex128
(a library routine) on the same values; bars: fp32 relative Frobenius
<= 1e-5, fp64 <= 1e-12.
"""
import numpy as np
import pytest

import einsum_ir_amd as eir
from einsum_ir_amd import host
from tests.helpers import TOL_FP32, TOL_FP64, rel_frobenius

pytestmark = pytest.mark.gpu


def _cpx(rng, shape, npt):
    return (rng.uniform(-1, 1, shape) + 1j * rng.uniform(-1, 1, shape)).astype(
        np.complex64 if npt == np.float32 else np.complex128)


def _planar(z):
    """complex array -> float array with an outermost dim of size 2 (re, im)"""
    return np.ascontiguousarray(np.stack([z.real, z.imag]))


def _from_planar(x):
    return x[0] + 1j * x[1]


@pytest.mark.parametrize("npt", [np.float32, np.float64])
@pytest.mark.parametrize("layout", ["inner", "outer"])
@pytest.mark.parametrize("accumulate", [False, True])
def test_cpx_matmul_plan(torch_cuda, npt, layout, accumulate):
    """km,nk->nm with the complex dim innermost (interleaved) or outermost
    (planar); first touch CPX_ZERO or UNDEFINED (accumulate)."""
    torch = torch_cuda
    m, n, k = 70, 52, 37
    rng = np.random.default_rng(11)
    A, B, O0 = _cpx(rng, (k, m), npt), _cpx(rng, (n, k), npt), _cpx(rng, (n, m), npt)
    if layout == "inner":
        # element (.., c): strides as the real view of the complex array
        a, b, o = A.view(npt).reshape(-1), B.view(npt).reshape(-1), O0.view(npt).reshape(-1).copy()
        sc = (1, 1, 1)
        sa = dict(k=2 * m, m=2)
        sb = dict(n=2 * k, k=2)
        so = dict(n=2 * m, m=2)
    else:
        a, b, o = _planar(A).reshape(-1), _planar(B).reshape(-1), _planar(O0).reshape(-1).copy()
        sc = (k * m, n * k, n * m)
        sa = dict(k=m, m=1)
        sb = dict(n=k, k=1)
        so = dict(n=m, m=1)
    # loops: cpx, m, n, k
    types = [eir.DIM_CPX, eir.DIM_M, eir.DIM_N, eir.DIM_K]
    sizes = [2, m, n, k]
    sl = [sc[0], sa["m"], 0, sa["k"]]
    sr = [sc[1], 0, sb["n"], sb["k"]]
    so_ = [sc[2], so["m"], so["n"], 0]
    dt = eir.FP32 if npt == np.float32 else eir.FP64
    plan = eir.ContractionPlan(types, sizes, sl, sr, so_, dtype_left=dt, dtype_right=dt, dtype_comp=dt,
                               dtype_out=dt,
                               ktype_first_touch=eir.UNDEFINED_KTYPE if accumulate else eir.CPX_ZERO,
                               ktype_main=eir.CPX_MADD)
    assert "cpx_" in plan.describe()
    da, db, do = (torch.from_numpy(x).cuda() for x in (a, b, o))
    plan.execute(da, db, do)
    torch.cuda.synchronize()
    got = do.cpu().numpy()
    got = got.view(A.dtype).reshape(n, m) if layout == "inner" else _from_planar(got.reshape(2, n, m))
    ref = np.einsum("km,nk->nm", A.astype(np.complex128), B.astype(np.complex128))
    if accumulate:
        ref = ref + O0
    tol = TOL_FP32 if npt == np.float32 else TOL_FP64
    assert rel_frobenius(ref, got) <= tol
    plan.close()


def test_cpx_vector_loads_batched(torch_cuda):
    """Planar complex with unit-stride M/N and K: the 16-byte vector loaders
    run for both parts; a C dim and a multi-dim K."""
    torch = torch_cuda
    z, m, n, k1, k2 = 3, 64, 48, 8, 6
    rng = np.random.default_rng(12)
    A = _cpx(rng, (z, k1, k2, m), np.float32)
    B = _cpx(rng, (z, n, k1, k2), np.float32)
    a, b = _planar(A).reshape(-1), _planar(B).reshape(-1)
    o = np.zeros(2 * z * n * m, np.float32)
    types = [eir.DIM_CPX, eir.DIM_C, eir.DIM_M, eir.DIM_N, eir.DIM_K, eir.DIM_K]
    sizes = [2, z, m, n, k1, k2]
    sl = [z * k1 * k2 * m, k1 * k2 * m, 1, 0, k2 * m, m]
    sr = [z * n * k1 * k2, n * k1 * k2, 0, k1 * k2, k2, 1]
    so = [z * n * m, n * m, 1, m, 0, 0]
    plan = eir.ContractionPlan(types, sizes, sl, sr, so, ktype_first_touch=eir.CPX_ZERO, ktype_main=eir.CPX_MADD)
    desc = plan.describe()
    assert "vec" in desc, desc
    do = torch.from_numpy(o).cuda()
    plan.execute(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda(), do)
    torch.cuda.synchronize()
    got = _from_planar(do.cpu().numpy().reshape(2, z, n, m))
    ref = np.einsum("zijm,znij->znm", A.astype(np.complex128), B.astype(np.complex128))
    assert rel_frobenius(ref, got) <= TOL_FP32
    plan.close()


def test_cpx_plan_errors(torch_cuda):
    types = [eir.DIM_CPX, eir.DIM_M, eir.DIM_N, eir.DIM_K]
    ok = dict(dtype_left=eir.FP32, dtype_right=eir.FP32)
    with pytest.raises(eir.EinsumIrError) as e:     # complex loop of size 3
        eir.ContractionPlan(types, [3, 4, 4, 4], [16, 1, 0, 4], [16, 0, 4, 1], [16, 1, 4, 0],
                            ktype_first_touch=eir.CPX_ZERO, ktype_main=eir.CPX_MADD, **ok)
    assert e.value.code == eir.INVALID_CPX_DIM
    with pytest.raises(eir.EinsumIrError) as e:     # complex loop with a real kernel
        eir.ContractionPlan(types, [2, 4, 4, 4], [16, 1, 0, 4], [16, 0, 4, 1], [16, 1, 4, 0], **ok)
    assert e.value.code == eir.INVALID_CPX_DIM
    with pytest.raises(eir.EinsumIrError) as e:     # bf16 complex
        eir.ContractionPlan(types, [2, 4, 4, 4], [16, 1, 0, 4], [16, 0, 4, 1], [16, 1, 4, 0],
                            dtype_left=eir.BF16, dtype_right=eir.BF16,
                            ktype_first_touch=eir.CPX_ZERO, ktype_main=eir.CPX_MADD)
    assert e.value.code == eir.INVALID_DTYPE


def test_expression_batch_inner_matmul(torch_cuda):
    """The reference's "single batch-inner complex matmul" (kmc,nkc->nmc,
    EinsumExpression.test.torch.cpp:150-205), including its num_ops."""
    torch = torch_cuda
    rng = np.random.default_rng(13)
    A, B = _cpx(rng, (4, 2), np.float32), _cpx(rng, (3, 4), np.float32)
    da, db = torch.from_numpy(A).cuda(), torch.from_numpy(B).cuda()
    dout = torch.zeros((3, 2), dtype=torch.complex64, device="cuda")
    e = host.Expression("km,nk->nm", dict(k=4, m=2, n=3), [(0, 1)], [da, db, dout], ctype=host.BATCH_INNER)
    e.eval()
    ref = np.einsum("km,nk->nm", A.astype(np.complex128), B.astype(np.complex128))
    assert rel_frobenius(ref, dout.cpu().numpy()) <= TOL_FP32
    assert e.num_ops() == 4 * 2 * 3 * 4 * 2 - 2 * 2 * 3
    e.close()


@pytest.mark.parametrize("npt", [np.float32, np.float64])
def test_expression_batch_inner_tree(torch_cuda, npt):
    """A three-node complex tree with permuted inputs (complex64/complex128 tensors)."""
    torch = torch_cuda
    expr, sizes, path = "iae,bf,dcba,cg,dh->hgfei", dict(a=2, b=3, c=4, d=5, e=6, f=7, g=8, h=9, i=10), \
        [(1, 2), (0, 2), (0, 2), (0, 1)]
    rng = np.random.default_rng(14)
    ins, out = expr.split("->")
    arrays = [_cpx(rng, [sizes[d] for d in t], npt) for t in ins.split(",")]
    dev = [torch.from_numpy(x).cuda() for x in arrays]
    dout = torch.zeros([sizes[d] for d in out], dtype=dev[0].dtype, device="cuda")
    e = host.Expression(expr, sizes, path, dev + [dout], dtype=eir.FP32 if npt == np.float32 else eir.FP64,
                        ctype=host.BATCH_INNER)
    e.eval()
    ref = np.einsum(expr, *[x.astype(np.complex128) for x in arrays])
    assert rel_frobenius(ref, dout.cpu().numpy()) <= (TOL_FP32 if npt == np.float32 else TOL_FP64)
    e.close()


def test_expression_batch_outer(torch_cuda):
    """BATCH_OUTER: every tensor planar (all real parts, then all imaginary parts)."""
    torch = torch_cuda
    expr, sizes, path = "da,dce,bec->abc", dict(a=3, b=4, c=5, d=6, e=7), [(1, 2), (0, 1)]
    rng = np.random.default_rng(15)
    ins, out = expr.split("->")
    arrays = [_cpx(rng, [sizes[d] for d in t], np.float32) for t in ins.split(",")]
    dev = [torch.from_numpy(_planar(x)).cuda() for x in arrays]
    dout = torch.zeros([2] + [sizes[d] for d in out], device="cuda")
    e = host.Expression(expr, sizes, path, dev + [dout], ctype=host.BATCH_OUTER)
    e.eval()
    ref = np.einsum(expr, *[x.astype(np.complex128) for x in arrays])
    assert rel_frobenius(ref, _from_planar(dout.cpu().numpy())) <= TOL_FP32
    e.close()
