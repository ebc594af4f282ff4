"""GPU parity of the 8-byte vector load modes of the generic fp32 tiles
(vec8_mn: two consecutive rows, vec8_k: two consecutive k).  The planner picks
them where an operand's unit-stride run has even length that is not a
multiple of 4, so 16-byte vectors do not fit (the odd mode sizes times 2 of
the einsum_benchmark networks).  Checker: the CPU oracle (fp64 accumulation)
on the same seeded inputs, relative Frobenius error <= 1e-5."""
import numpy as np
import pytest

import einsum_ir_amd as eir
from tests.helpers import TOL_FP32, loops_for, parse_binary, rel_frobenius, tensor_numel
from tests.test_gpu_contract import run_case

pytestmark = pytest.mark.gpu

VEC8_SHAPES = [
    # expr, sizes, expected "A=..:mode B=..:mode" fragment
    ("km,kn->mn", dict(k=50, m=66, n=130), "A=left:vec8_mn B=right:vec8_mn"),
    ("mk,nk->mn", dict(m=70, k=54, n=90), "A=left:vec8_k B=right:vec8_k"),
    ("km,nk->mn", dict(k=38, m=134, n=70), "A=left:vec8_mn B=right:vec8_k"),
    ("mk,kn->mn", dict(m=70, k=46, n=258), "A=left:vec8_k B=right:vec8_mn"),
    ("km,kn->mn", dict(k=40, m=64, n=70), "A=left:vec_mn B=right:vec8_mn"),
    ("zkm,zkn->zmn", dict(z=3, k=22, m=66, n=34), "A=left:vec8_mn B=right:vec8_mn"),
    # K over two dims, unit-stride in A only: A vec8_k with the K table
    # (not affine), B gathered
    ("mkl,nlk->mn", dict(m=66, k=5, l=6, n=36), "A=left:vec8_k B=right:scalar"),
    # K shorter than one k step, ragged M and N
    ("mk,nk->mn", dict(m=150, k=6, n=98), "A=left:vec8_k B=right:vec8_k"),
]


@pytest.mark.parametrize("tile", [None, "0", "1"])
@pytest.mark.parametrize("expr,sizes,modes", VEC8_SHAPES)
def test_vec8_modes(torch_cuda, oracle, monkeypatch, expr, sizes, modes, tile):
    if tile is None:
        monkeypatch.delenv("ETIR_TILE", raising=False)
    else:
        monkeypatch.setenv("ETIR_TILE", tile)
    _, desc = run_case(torch_cuda, oracle, expr, sizes, seed=len(expr) + sum(sizes.values()))
    assert modes in desc, desc
    if tile is not None:
        assert ("f32_128x128" if tile == "0" else "f32_64x64") in desc, desc


@pytest.mark.parametrize("first,last", [(eir.COPY, eir.RELU), (eir.ADD, eir.UNDEFINED_KTYPE),
                                        (eir.UNDEFINED_KTYPE, eir.ADD)])
def test_vec8_touch_kernels(torch_cuda, oracle, first, last):
    _, desc = run_case(torch_cuda, oracle, "km,nk->mn", dict(k=38, m=134, n=70), first=first, last=last,
                       seed=first * 3 + last)
    assert "vec8" in desc, desc


def test_vec8_misaligned_pointer_falls_back(torch_cuda, oracle):
    """An operand 4 bytes off an 8-byte boundary cannot take 8-byte vectors:
    the launch gathers it element by element instead (same results)."""
    torch = torch_cuda
    expr, sizes = "mk,nk->mn", dict(m=70, k=54, n=90)
    left, right, out = parse_binary(expr)
    loops = loops_for(expr, sizes)
    rng = np.random.default_rng(5)
    a = rng.uniform(-1, 1, tensor_numel(left, sizes)).astype(np.float32)
    b = rng.uniform(-1, 1, tensor_numel(right, sizes)).astype(np.float32)
    plan = eir.ContractionPlan(loops["dim_types"], loops["sizes"], loops["strides_left"],
                               loops["strides_right"], loops["strides_out"])
    assert "vec8_k" in plan.describe()
    buf_a = torch.zeros(a.size + 1, device="cuda")
    buf_a[1:] = torch.from_numpy(a).cuda()
    db = torch.from_numpy(b).cuda()
    do = torch.zeros(tensor_numel(out, sizes), device="cuda")
    plan.execute(buf_a[1:], db, do, stream=torch.cuda.current_stream())
    torch.cuda.synchronize()
    plan.close()
    ref = np.zeros(tensor_numel(out, sizes), dtype=np.float32)
    oracle.contract(loops, a, b, ref)
    assert rel_frobenius(ref, do.cpu().numpy()) <= TOL_FP32
