"""GPU parity of the fp32 contraction that splits K over the waves of one
workgroup (tile f32_kwave_32x32): few output tiles, both operands
K-contiguous.  Ragged tile edges, C dims, a non-affine row table, K over
several register batches, every touch kernel.  Checker: the CPU oracle (fp64
accumulation), relative Frobenius error <= 1e-5."""
import numpy as np
import pytest

import einsum_ir_amd as eir
from tests.test_gpu_contract import run_case

pytestmark = pytest.mark.gpu

KWAVE_SHAPES = [
    ("mk,nk->mn", dict(m=390, n=356, k=512)),          # ragged edges, BASELINE-1-like K
    ("cmk,cnk->cmn", dict(c=3, m=224, n=200, k=256)),   # C dims
    ("abk,nk->ban", dict(a=12, b=24, n=480, k=256)),    # kernel rows (b, a): non-affine A row table
    ("mk,nk->mn", dict(m=400, n=360, k=4096)),          # four register batches per wave
    ("abkl,cdkl->abcd", dict(a=32, b=16, c=32, d=16, k=32, l=16)),
]


@pytest.mark.parametrize("expr,sizes", KWAVE_SHAPES)
def test_kwave_layouts(torch_cuda, oracle, expr, sizes):
    _, desc = run_case(torch_cuda, oracle, expr, sizes, seed=31)
    assert "f32_kwave_32x32" in desc, desc


@pytest.mark.parametrize("first,last", [(eir.COPY, eir.UNDEFINED_KTYPE), (eir.ADD, eir.UNDEFINED_KTYPE),
                                        (eir.UNDEFINED_KTYPE, eir.UNDEFINED_KTYPE), (eir.ZERO, eir.RELU),
                                        (eir.COPY, eir.RELU), (eir.ZERO, eir.ADD)])
def test_kwave_touch_kernels(torch_cuda, oracle, first, last):
    _, desc = run_case(torch_cuda, oracle, "mk,nk->mn", dict(m=390, n=356, k=256), first=first, last=last,
                       seed=37)
    assert "f32_kwave_32x32" in desc, desc


def test_kwave_matches_split_k(torch_cuda, oracle, monkeypatch):
    """The same contraction through the workgroup K split and through split K."""
    got_w, desc_w = run_case(torch_cuda, oracle, "mk,nk->mn", dict(m=256, n=512, k=1024), seed=41)
    monkeypatch.setenv("ETIR_NO_KWAVE", "1")
    got_s, desc_s = run_case(torch_cuda, oracle, "mk,nk->mn", dict(m=256, n=512, k=1024), seed=41)
    assert "kwave" in desc_w and "kwave" not in desc_s, (desc_w, desc_s)
    assert np.linalg.norm(got_w - got_s) / np.linalg.norm(got_s) <= 1e-5
