"""GPU parity of fp64 contractions (tile f64_64x64x16, v_mfma_f64_16x16x4_f64):
the reference's FP64 data type on its binary-contraction path (reference
src/backend/BinaryContractionTpp.test.torch.cpp:442-510 "matmuls with FP64
and zero first touch", EinsumExpression/EinsumTree FP64 cases).  Every load
mode of both operands, table and affine K, K not a multiple of the k step,
ragged M/N edges, C dims, and every touch kernel.  Checker: the CPU oracle
(fp64 accumulation) on identical seeded inputs; bar: relative Frobenius
error <= 1e-12 (the two sums differ only in order)."""
import numpy as np
import pytest

import einsum_ir_amd as eir
from tests.helpers import TOL_FP64, rel_frobenius, loops_for
from tests.test_gpu_contract import run_case

pytestmark = pytest.mark.gpu

F64_SHAPES = [
    # (expression, sizes, load modes expected in the plan description)
    ("km,nk->nm", dict(k=4, m=2, n=3), None),                                # the reference's FP64 case
    ("mk,kn->mn", dict(m=100, k=37, n=70), "A=left:scalar B=right:vec_mn"),   # odd row stride: gathers
    ("mk,kn->mn", dict(m=100, k=38, n=70), "A=left:vec_k B=right:vec_mn"),
    ("km,kn->mn", dict(k=50, m=96, n=130), "vec_mn"),
    ("mk,nk->mn", dict(m=65, k=64, n=66), "vec_k"),
    ("abkl,cdkl->abcd", dict(a=8, b=6, c=5, d=7, k=9, l=4), None),           # multi-mode, odd sizes
    ("zakm,zbkn->zabmn", dict(z=2, a=3, m=16, b=2, n=16, k=40), "vec_mn"),  # config-3 layout, small
    ("ikj,jkl->il", dict(i=33, j=7, k=5, l=29), None),                       # non-affine K (k, j split)
]


@pytest.mark.parametrize("expr,sizes,modes", F64_SHAPES)
def test_f64_layouts(torch_cuda, oracle, expr, sizes, modes):
    _, desc = run_case(torch_cuda, oracle, expr, sizes, dtype=eir.FP64, seed=len(expr))
    assert "f64_64x64x16" in desc, desc
    if modes:
        for m in modes.split():
            assert m in desc, desc


@pytest.mark.parametrize("first,last", [(eir.COPY, eir.UNDEFINED_KTYPE), (eir.ADD, eir.UNDEFINED_KTYPE),
                                        (eir.UNDEFINED_KTYPE, eir.UNDEFINED_KTYPE), (eir.ZERO, eir.RELU),
                                        (eir.COPY, eir.RELU), (eir.ZERO, eir.ADD)])
def test_f64_touch_kernels(torch_cuda, oracle, first, last):
    run_case(torch_cuda, oracle, "mk,kn->mn", dict(m=70, k=33, n=90), dtype=eir.FP64,
             first=first, last=last, seed=5)


@pytest.mark.parametrize("bcast", ["row", "col", "scalar"])
def test_f64_bias_broadcast(torch_cuda, oracle, bcast):
    """bias COPY broadcast through aux outer sizes of 1 (BinaryContractionTpp.test.torch.cpp:77-367)."""
    aux = dict(m=64, n=48, k=32)
    if bcast in ("row", "scalar"):
        aux["m"] = 1
    if bcast in ("col", "scalar"):
        aux["n"] = 1
    run_case(torch_cuda, oracle, "mk,kn->mn", dict(m=64, k=32, n=48), dtype=eir.FP64,
             first=eir.COPY, last=eir.RELU, aux_outer=aux, seed=6)


def test_f64_long_k_no_split(torch_cuda, oracle):
    """Few tiles and a long K: fp64 stays one launch (the split-K workspace is fp32)."""
    _, desc = run_case(torch_cuda, oracle, "mk,kn->mn", dict(m=64, k=4096, n=64), dtype=eir.FP64, seed=7)
    assert "split" not in desc


def test_f64_tree(torch_cuda, oracle):
    """An FP64 einsum tree (reference EinsumTree.test.torch.cpp:131 uses FP64)."""
    from einsum_ir_amd import host
    torch = torch_cuda
    expr, sizes, path = "da,dce,bec->abc", dict(a=3, b=4, c=5, d=6, e=7), [(1, 2), (0, 1)]
    rng = np.random.default_rng(9)
    ins = expr.split("->")[0].split(",")
    arrays = [rng.uniform(-1, 1, int(np.prod([sizes[d] for d in t]))) for t in ins]
    dev = [torch.from_numpy(x).cuda() for x in arrays]
    dout = torch.zeros(3 * 4 * 5, dtype=torch.float64, device="cuda")
    e = host.Expression(expr, sizes, path, dev + [dout], dtype=eir.FP64)
    e.eval()
    ops = [x.reshape([sizes[d] for d in t]) for x, t in zip(arrays, ins)]
    ref = np.einsum(expr, *ops)
    assert rel_frobenius(ref, dout.cpu().numpy().reshape(3, 4, 5)) <= TOL_FP64
    e.close()
