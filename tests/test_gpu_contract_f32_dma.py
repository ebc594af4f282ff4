"""GPU parity of the fp32 direct-to-LDS contraction kernel (tile
f32_dma_128x128x32): every load-mode pairing, ragged M/N edges, K that is not
a multiple of the k step, K through offset tables, C dims, the touch kernels,
the split-K partials it
runs for few tiles and a long K; and the launch-time fallback of every
vector-only kernel (fp32 and bf16 direct-to-LDS, K over waves) to the
register-staged kernel when an operand pointer is not 16-byte aligned.
Checker: the CPU oracle (fp64 accumulation) on the same inputs, relative
Frobenius error <= 1e-5 (fp32) / 2e-3 (bf16)."""
import numpy as np
import pytest

import einsum_ir_amd as eir
from tests.helpers import loops_for, parse_binary, rel_frobenius, tensor_numel
from tests.test_gpu_contract import TOL_BF16, TOL_FP32, run_case

pytestmark = pytest.mark.gpu

F32_DMA_SHAPES = [
    ("km,kn->mn", dict(k=136, m=264, n=520)),                              # ragged M and N, K % 32 != 0
    ("zakm,zbkn->zabmn", dict(z=2, a=3, m=64, b=5, n=64, k=200)),          # C dims, two-dim M and N
    ("mk,nk->mn", dict(m=300, k=72, n=260)),                               # K-contiguous operands
    ("km,nk->mn", dict(k=40, m=136, n=264)),
    ("mk,kn->mn", dict(m=264, k=104, n=136)),
    ("mk,kn->mn", dict(m=8, k=8, n=8)),                                    # one partial tile
    ("km,kn->mn", dict(k=2048, m=512, n=384)),                             # 64 k steps
]


@pytest.mark.parametrize("expr,sizes", F32_DMA_SHAPES)
def test_f32_dma_layouts(torch_cuda, oracle, monkeypatch, expr, sizes):
    monkeypatch.setenv("ETIR_TILE", "12")
    _, desc = run_case(torch_cuda, oracle, expr, sizes, seed=len(expr) + sizes["k"])
    assert "f32_dma_128x128x32" in desc, desc


@pytest.mark.parametrize("k", [4, 20, 36, 44, 56, 88])
@pytest.mark.parametrize("expr", ["km,kn->mn", "mk,nk->mn"])
def test_f32_dma_k_tail(torch_cuda, oracle, monkeypatch, expr, k):
    """The last k step skips its fragment steps wholly past K (4, 20, 4, 12,
    24 and 24 valid k of 32 in its last step), both operand orientations
    (K a multiple of 4 keeps K-contiguous rows 16-byte loadable)."""
    monkeypatch.setenv("ETIR_TILE", "12")
    _, desc = run_case(torch_cuda, oracle, expr, dict(k=k, m=136, n=264), seed=k)
    assert "f32_dma_128x128x32" in desc, desc


# K of two dims whose strides make it affine for one operand only: the K
# offsets come from the plan's tables (staged in LDS by the kernel)
F32_DMA_TABLE_K = [
    ("klm,lkn->mn", dict(k=8, l=16, m=264, n=520)),                        # vec_mn x vec_mn
    ("mkl,lkn->mn", dict(m=300, k=16, l=8, n=260)),                        # vec_k x vec_mn
    ("klm,nlk->mn", dict(k=12, l=8, m=136, n=264)),
    ("zklm,zlkn->zmn", dict(z=3, k=4, l=36, m=128, n=128)),                # K = 144, C dim
]


@pytest.mark.parametrize("expr,sizes", F32_DMA_TABLE_K)
def test_f32_dma_table_k(torch_cuda, oracle, monkeypatch, expr, sizes):
    monkeypatch.setenv("ETIR_TILE", "12")
    _, desc = run_case(torch_cuda, oracle, expr, sizes, seed=sum(sizes.values()))
    assert "f32_dma_128x128x32" in desc and "k_affine=0" in desc, desc


@pytest.mark.parametrize("first,last", [(eir.COPY, eir.UNDEFINED_KTYPE), (eir.ADD, eir.UNDEFINED_KTYPE),
                                        (eir.UNDEFINED_KTYPE, eir.UNDEFINED_KTYPE), (eir.ZERO, eir.RELU),
                                        (eir.COPY, eir.RELU), (eir.ZERO, eir.ADD)])
def test_f32_dma_touch_kernels(torch_cuda, oracle, monkeypatch, first, last):
    monkeypatch.setenv("ETIR_TILE", "12")
    _, desc = run_case(torch_cuda, oracle, "km,kn->mn", dict(k=96, m=272, n=264), first=first, last=last)
    assert "f32_dma_128x128x32" in desc


def test_f32_dma_split_k(torch_cuda, oracle, monkeypatch):
    """Few tiles and a long K: the planner splits K; the partial contraction
    runs on the fp32 DMA kernel (forced: left alone the planner gives the
    partial the 64 x 64 tile for more workgroups) and the reduction adds the
    slices."""
    monkeypatch.setenv("ETIR_TILE", "12")
    _, desc = run_case(torch_cuda, oracle, "km,kn->mn", dict(k=8192, m=256, n=256), seed=5)
    assert "split" in desc and "f32_dma_128x128x32" in desc, desc


def test_f32_dma_is_the_default_for_large_fp32(torch_cuda):
    """The planner takes the fp32 DMA kernel where it chose the 128 x 128
    fp32 tile (here a node of BASELINE config 4); other shapes keep theirs."""
    for expr, sizes, want in [("bi,ih->bh", dict(b=4096, i=2048, h=2048), "f32_dma_128x128x32"),
                              ("mk,kn->mn", dict(m=64, k=64, n=64), "f32_64x64x32")]:
        loops = loops_for(expr, sizes)
        plan = eir.ContractionPlan(loops["dim_types"], loops["sizes"], loops["strides_left"],
                                   loops["strides_right"], loops["strides_out"])
        desc = plan.describe()
        plan.close()
        assert want in desc, (expr, desc)


def _run_offset(torch, oracle, expr, sizes, dtype, tile, seed=0):
    """Plans the contraction, then executes it on operands whose device
    pointers are one element past a 256-byte boundary (not 16-byte aligned):
    the kernels that need 16-byte vectors must hand over to the
    register-staged kernel with gathers and give the same result."""
    left, right, out = parse_binary(expr)
    loops = loops_for(expr, sizes)
    rng = np.random.default_rng(seed)
    a = rng.uniform(-1, 1, tensor_numel(left, sizes)).astype(np.float32)
    b = rng.uniform(-1, 1, tensor_numel(right, sizes)).astype(np.float32)
    tdt = torch.float32
    if dtype == eir.BF16:
        a, b = oracle.f32_to_bf16(a), oracle.f32_to_bf16(b)
        tdt = torch.int16

    def offset_dev(x):
        host = torch.from_numpy(x.view(np.int16) if x.dtype == np.uint16 else x)
        buf = torch.zeros(x.size + 64, dtype=tdt, device="cuda")
        view = buf[1:1 + x.size]
        view.copy_(host.cuda())
        assert view.data_ptr() % 16 != 0
        return buf, view

    plan = eir.ContractionPlan(loops["dim_types"], loops["sizes"], loops["strides_left"],
                               loops["strides_right"], loops["strides_out"], dtype_left=dtype, dtype_right=dtype)
    desc = plan.describe()
    assert tile in desc, desc
    ba, da = offset_dev(a)
    bb, db = offset_dev(b)
    do = torch.zeros(tensor_numel(out, sizes), dtype=torch.float32, device="cuda")
    plan.execute(da, db, do, stream=torch.cuda.current_stream())
    torch.cuda.synchronize()
    got = do.cpu().numpy()
    plan.close()
    ref = np.zeros(tensor_numel(out, sizes), dtype=np.float32)
    oracle.contract(loops, a, b, ref, dtype_left=dtype, dtype_right=dtype, dtype_out=eir.FP32)
    err = rel_frobenius(ref, got)
    tol = TOL_BF16 if dtype == eir.BF16 else TOL_FP32
    assert err <= tol, f"{expr} {sizes} ({tile}, unaligned operands): rel. Frobenius error {err:.3e}"


@pytest.mark.parametrize("expr,sizes,dtype,tile,force", [
    ("km,kn->mn", dict(k=136, m=264, n=520), eir.FP32, "f32_dma_128x128x32", "12"),   # falls back to 64 x 64
    ("bi,ih->bh", dict(b=2048, i=256, h=2048), eir.FP32, "f32_dma_128x128x32", None),  # ... to 128 x 128
    ("abkl,cdkl->abcd", dict(a=32, b=16, c=32, d=16, k=32, l=16), eir.FP32, "f32_kwave_32x32", None),
    ("zakm,zbkn->zabmn", dict(z=2, a=8, m=64, b=8, n=64, k=128), eir.BF16, "bf16_dma_256x256", "7"),
    ("zakm,zbkn->zabmn", dict(z=2, a=8, m=64, b=8, n=64, k=96), eir.BF16, "bf16_dma_256x128", "8"),
])
def test_unaligned_operands_fall_back(torch_cuda, oracle, monkeypatch, expr, sizes, dtype, tile, force):
    if force:
        monkeypatch.setenv("ETIR_TILE", force)
    _run_offset(torch_cuda, oracle, expr, sizes, dtype, tile, seed=sizes.get("k", 1))


@pytest.mark.parametrize("k,split", [(2048, "S=16 K'=128"), (2060, "S=5 K'=412"), (2053, None)])
def test_long_k_split_on_large_tiles(torch_cuda, oracle, monkeypatch, k, split):
    """K >= 2048 on fewer than 256 tiles of 128 x 128: the planner takes the
    fp32 direct-to-LDS tile split over K, with factors that keep the K rows
    16-byte loadable (2060 = 5 x 412, not 4 x 515; the partial contraction
    picks its own tile); a prime K does not split and the node stays on the
    64 x 64 tile."""
    monkeypatch.delenv("ETIR_TILE", raising=False)
    _, desc = run_case(torch_cuda, oracle, "mk,nk->mn", dict(m=264, k=k, n=200), seed=k)
    if split is None:
        assert "split-K" not in desc and "f32_64x64x32" in desc, desc
    else:
        assert split in desc, desc
