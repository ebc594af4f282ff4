"""GPU parity of the matrix-vector contraction kernel (tile "gemv": kernel
M == 1 or N == 1, one thread per output element): the planner's own choice
on shapes that fill the chip, and forced (ETIR_TILE=13) on small ones -- M == 1
and N == 1 (roles swapped), both at once, C dims, K through offset tables, K
below and above the 8-wide load chunk, ragged extents, bf16 inputs and
outputs, and every touch-kernel pairing.
Checker: the CPU oracle (fp64 accumulation) on the same inputs, relative
Frobenius error <= 1e-5 (fp32) / 2e-3 (bf16)."""
import pytest

import einsum_ir_amd as eir
from tests.test_gpu_contract import run_case

pytestmark = pytest.mark.gpu

# the planner picks the kernel by itself: outputs >= 256 x 1024, K <= 256,
# the long operand unit-stride along the long side
AUTO_SHAPES = [
    ("zk,zkn->zn", dict(z=64, k=11, n=8192)),             # M == 1, a batch of vector-matrix products
    ("zkm,zk->zm", dict(z=32, k=24, m=8200)),             # N == 1 on the left operand, ragged
    ("k,kn->n", dict(k=256, n=300000)),                   # one product, K at the limit
]


@pytest.mark.parametrize("expr,sizes", AUTO_SHAPES)
def test_gemv_auto(torch_cuda, oracle, monkeypatch, expr, sizes):
    monkeypatch.delenv("ETIR_TILE", raising=False)
    _, desc = run_case(torch_cuda, oracle, expr, sizes, seed=sizes["k"])
    assert "contract gemv" in desc, desc


def test_gemv_not_chosen_for_few_outputs(torch_cuda, oracle, monkeypatch):
    """Too few outputs to fill the chip with one thread each: the MFMA tiles."""
    monkeypatch.delenv("ETIR_TILE", raising=False)
    _, desc = run_case(torch_cuda, oracle, "k,kn->n", dict(k=64, n=4096), seed=3)
    assert "gemv" not in desc, desc


FORCED_SHAPES = [
    ("k,kn->n", dict(k=40, n=300)),
    ("kn,k->n", dict(k=5, n=77)),                          # K below one load chunk
    ("mk,k->m", dict(m=129, k=300)),                       # K-contiguous long operand
    ("k,mk->m", dict(m=1000, k=17)),
    ("zk,zk->z", dict(z=50, k=33)),                        # M == N == 1: one dot product per C index
    ("zk,kzn->zn", dict(z=3, k=9, n=70)),                  # a C dim at a different place in each tensor
    ("kmz,kz->mz", dict(z=3, k=10, m=200)),                # a C dim innermost in the output: N == 1
    ("lk,zkln->zn", dict(z=4, l=6, k=7, n=96)),            # K of two dims: offsets from tables
]


@pytest.mark.parametrize("expr,sizes", FORCED_SHAPES)
@pytest.mark.parametrize("dtype,dtype_out", [(eir.FP32, eir.FP32), (eir.BF16, eir.FP32), (eir.BF16, eir.BF16)])
def test_gemv_forced(torch_cuda, oracle, monkeypatch, expr, sizes, dtype, dtype_out):
    monkeypatch.setenv("ETIR_TILE", "13")
    _, desc = run_case(torch_cuda, oracle, expr, sizes, dtype=dtype, dtype_out=dtype_out,
                       seed=sum(sizes.values()))
    assert "contract gemv" in desc, desc


def test_gemv_table_k(torch_cuda, oracle, monkeypatch):
    monkeypatch.setenv("ETIR_TILE", "13")
    _, desc = run_case(torch_cuda, oracle, "lk,zkln->zn", dict(z=4, l=6, k=7, n=96), seed=11)
    assert "contract gemv" in desc and "k_affine=0" in desc, desc


@pytest.mark.parametrize("first,last", [(eir.ZERO, eir.UNDEFINED_KTYPE), (eir.COPY, eir.UNDEFINED_KTYPE),
                                        (eir.ADD, eir.UNDEFINED_KTYPE), (eir.UNDEFINED_KTYPE, eir.UNDEFINED_KTYPE),
                                        (eir.ZERO, eir.RELU), (eir.COPY, eir.RELU), (eir.ZERO, eir.ADD)])
@pytest.mark.parametrize("dtype_out", [eir.FP32, eir.BF16])
def test_gemv_touch_kernels(torch_cuda, oracle, monkeypatch, first, last, dtype_out):
    monkeypatch.setenv("ETIR_TILE", "13")
    dtype = eir.BF16 if dtype_out == eir.BF16 else eir.FP32
    _, desc = run_case(torch_cuda, oracle, "zk,zkn->zn", dict(z=3, k=20, n=200), dtype=dtype,
                       dtype_out=dtype_out, first=first, last=last, seed=first * 7 + last)
    assert "contract gemv" in desc, desc


def test_gemv_switched_off(torch_cuda, oracle, monkeypatch):
    monkeypatch.delenv("ETIR_TILE", raising=False)
    monkeypatch.setenv("ETIR_NO_GEMV", "1")
    _, desc = run_case(torch_cuda, oracle, "zk,zkn->zn", dict(z=64, k=11, n=8192), seed=2)
    assert "gemv" not in desc, desc


@pytest.mark.parametrize("dtype,dtype_out,first,last", [
    (eir.FP32, eir.FP32, eir.ZERO, eir.UNDEFINED_KTYPE),
    (eir.FP32, eir.FP32, eir.COPY, eir.RELU),
    (eir.FP32, eir.FP32, eir.ADD, eir.UNDEFINED_KTYPE),
    (eir.BF16, eir.FP32, eir.ZERO, eir.UNDEFINED_KTYPE),
    (eir.BF16, eir.BF16, eir.UNDEFINED_KTYPE, eir.ADD),
])
def test_gemv_four_outputs_per_thread(torch_cuda, oracle, monkeypatch, dtype, dtype_out, first, last):
    """Kernel M == 1 with the long operand and the output unit-stride along n
    ('v4': 4 outputs per thread, vector loads and stores) against the
    one-output kernel, which runs when the long operand's base address is not
    vector-aligned (offset by one element): the same bits, and the oracle's
    result.  K = 11 (one 8-wide chunk and a tail), a bias broadcast over the
    batch dim for the aux touches."""
    import numpy as np
    from tests.helpers import loops_for, rel_frobenius
    torch = torch_cuda
    monkeypatch.delenv("ETIR_TILE", raising=False)
    z, k, n = 64, 11, 8192
    loops = loops_for("zk,zkn->zn", dict(z=z, k=k, n=n), sizes_outer_aux=dict(z=1, n=n))
    rng = np.random.default_rng(80 + first + 10 * last)
    tdt = torch.bfloat16 if dtype == eir.BF16 else torch.float32
    odt = torch.bfloat16 if dtype_out == eir.BF16 else torch.float32
    a = torch.from_numpy(rng.uniform(-1, 1, z * k).astype(np.float32)).cuda().to(tdt)
    b0 = torch.from_numpy(rng.uniform(-1, 1, z * k * n).astype(np.float32)).cuda().to(tdt)
    b_all = torch.empty(z * k * n + 1, device="cuda", dtype=tdt)
    b_all[1:].copy_(b0)
    b1 = b_all[1:]                              # same values, base address one element off
    aux = torch.from_numpy(rng.uniform(-1, 1, n).astype(np.float32)).cuda().to(odt)
    o0 = torch.from_numpy(rng.uniform(-1, 1, z * n).astype(np.float32)).cuda().to(odt)
    plan = eir.ContractionPlan(loops["dim_types"], loops["sizes"], loops["strides_left"], loops["strides_right"],
                               loops["strides_out"], strides_out_aux=loops["strides_out_aux"], dtype_left=dtype,
                               dtype_right=dtype, dtype_out=dtype_out, ktype_first_touch=first,
                               ktype_last_touch=last)
    desc = plan.describe()
    assert "contract gemv" in desc and " v4" in desc, desc
    outs = []
    for b in (b0, b1):
        o = o0.clone()
        plan.execute(a, b, o, aux=aux, stream=torch.cuda.current_stream())
        torch.cuda.synchronize()
        outs.append(o.float().cpu().numpy())
    plan.close()
    assert np.array_equal(outs[0], outs[1]), "4-output and 1-output kernels differ"
    A = a.float().double().cpu().numpy().reshape(z, k)
    B = b0.float().double().cpu().numpy().reshape(z, k, n)
    ref = np.einsum("zk,zkn->zn", A, B)
    x = aux.float().double().cpu().numpy().reshape(1, n)
    old = o0.float().double().cpu().numpy().reshape(z, n)
    if first == eir.COPY:
        ref = ref + x
    elif first == eir.ADD:
        ref = ref + x + old
    elif first == eir.UNDEFINED_KTYPE:
        ref = ref + old
    if last == eir.RELU:
        ref = np.maximum(ref, 0.0)
    elif last == eir.ADD:
        ref = ref + x
    tol = 2e-3 if (dtype == eir.BF16 or dtype_out == eir.BF16) else 1e-5
    assert rel_frobenius(ref.ravel(), outs[0].ravel()) <= tol
