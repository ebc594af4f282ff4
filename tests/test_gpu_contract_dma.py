"""GPU parity of the direct-to-LDS bf16 contraction kernel (tile
bf16_dma_256x256): every load-mode pairing, ragged M/N edges, K that is not a
multiple of the k step, both pipeline variants, the touch kernels and bf16
output.  Checker: the CPU oracle (fp64 accumulation) on the same bf16-rounded
inputs, relative Frobenius error <= 2e-3."""
import pytest

import einsum_ir_amd as eir
from tests.test_gpu_contract import run_case

pytestmark = pytest.mark.gpu

DMA_SHAPES = [
    ("km,kn->mn", dict(k=136, m=264, n=520), "A=left:vec_mn B=right:vec_mn"),
    ("zakm,zbkn->zabmn", dict(z=2, a=3, m=64, b=5, n=64, k=200), "A=left:vec_mn B=right:vec_mn"),
    ("mk,nk->mn", dict(m=300, k=72, n=260), "A=left:vec_k B=right:vec_k"),
    ("km,nk->mn", dict(k=40, m=136, n=264), "A=left:vec_mn B=right:vec_k"),
    ("mk,kn->mn", dict(m=264, k=104, n=136), "A=left:vec_k B=right:vec_mn"),
    ("mk,kn->mn", dict(m=8, k=8, n=8), "A=left:vec_k B=right:vec_mn"),
]


@pytest.mark.parametrize("variant", ["0", "1"])
@pytest.mark.parametrize("expr,sizes,modes", DMA_SHAPES)
def test_dma_layouts(torch_cuda, oracle, monkeypatch, expr, sizes, modes, variant):
    monkeypatch.setenv("ETIR_TILE", "7")
    monkeypatch.setenv("ETIR_DMA_VARIANT", variant)
    _, desc = run_case(torch_cuda, oracle, expr, sizes, dtype=eir.BF16, seed=len(expr) + int(variant))
    assert "bf16_dma_256x256" in desc and modes in desc, desc


@pytest.mark.parametrize("expr,sizes", [("km,kn->mn", dict(k=136, m=264, n=520)),
                                        ("zakm,zbkn->zabmn", dict(z=2, a=3, m=64, b=5, n=64, k=200))])
def test_dma_256x128_two_per_cu(torch_cuda, oracle, monkeypatch, expr, sizes):
    monkeypatch.setenv("ETIR_TILE", "8")
    _, desc = run_case(torch_cuda, oracle, expr, sizes, dtype=eir.BF16, seed=17)
    assert "bf16_dma_256x128" in desc, desc


@pytest.mark.parametrize("first,last", [(eir.COPY, eir.UNDEFINED_KTYPE), (eir.ADD, eir.UNDEFINED_KTYPE),
                                        (eir.UNDEFINED_KTYPE, eir.UNDEFINED_KTYPE), (eir.ZERO, eir.RELU),
                                        (eir.COPY, eir.RELU), (eir.ZERO, eir.ADD)])
def test_dma_touch_kernels(torch_cuda, oracle, monkeypatch, first, last):
    monkeypatch.setenv("ETIR_TILE", "7")
    _, desc = run_case(torch_cuda, oracle, "km,kn->mn", dict(k=96, m=272, n=264), dtype=eir.BF16,
                       first=first, last=last)
    assert "bf16_dma_256x256" in desc


def test_dma_bf16_output(torch_cuda, oracle, monkeypatch):
    monkeypatch.setenv("ETIR_TILE", "7")
    _, desc = run_case(torch_cuda, oracle, "km,kn->mn", dict(k=128, m=256, n=264), dtype=eir.BF16,
                       dtype_out=eir.BF16)
    assert "bf16_dma_256x256" in desc


def test_dma_is_the_default_for_c3(torch_cuda):
    """The planner picks the DMA kernel for BASELINE config 3 (2048 tiles of
    256 x 256); the full-size run is checked in test_gpu_contract."""
    from tests.helpers import loops_for
    loops = loops_for("zakm,zbkn->zabmn", dict(z=8, a=64, m=64, b=64, n=64, k=1024))
    plan = eir.ContractionPlan(loops["dim_types"], loops["sizes"], loops["strides_left"],
                               loops["strides_right"], loops["strides_out"], dtype_left=eir.BF16,
                               dtype_right=eir.BF16)
    desc = plan.describe()
    plan.close()
    assert "bf16_dma_256x256" in desc, desc


PERSISTENT_SHAPES = [
    # fewer tiles than CUs, not a multiple of 8: one tile per workgroup, plain tile order
    ("km,kn->mn", dict(k=136, m=512, n=768)),
    ("zakm,zbkn->zabmn", dict(z=3, a=4, m=64, b=8, n=64, k=72)),
    # 320 tiles over 256 workgroups (XCD ranges of 40 tiles, 32 workgroups
    # each: some workgroups run two tiles), K not a multiple of the k step
    ("zkm,zkn->zmn", dict(z=5, k=40, m=2048, n=2048)),
]


@pytest.mark.parametrize("expr,sizes", PERSISTENT_SHAPES)
def test_dma_persistent(torch_cuda, oracle, monkeypatch, expr, sizes):
    """The persistent variant (default for VEC_MN x VEC_MN with all tiles
    full, ZERO first touch, no last touch) against the oracle, and bit for bit
    against the one-tile-per-workgroup kernel: both sum each output in the
    same order, so any tile placed or walked wrongly shows up exactly."""
    monkeypatch.setenv("ETIR_TILE", "7")
    monkeypatch.delenv("ETIR_DMA_VARIANT", raising=False)
    got_p, desc = run_case(torch_cuda, oracle, expr, sizes, dtype=eir.BF16, seed=23)
    assert "bf16_dma_256x256" in desc and "persistent" in desc, desc
    monkeypatch.setenv("ETIR_DMA_VARIANT", "1")
    got_1, desc1 = run_case(torch_cuda, oracle, expr, sizes, dtype=eir.BF16, seed=23, check=False)
    assert "persistent" not in desc1, desc1
    assert (got_p == got_1).all(), "persistent and one-tile-per-workgroup kernels differ"


@pytest.mark.parametrize("variant,persistent", [("0", False), ("1", False), ("2", True), ("3", True),
                                                ("9", True)])
def test_dma_variant_override(torch_cuda, oracle, monkeypatch, variant, persistent):
    """ETIR_DMA_VARIANT takes only the values a 256 x 256 plan can run (0: BK 64
    loop, 1: one-tile scheduled loop, 3: persistent); others (2, the 256 x 128
    kernel with a tile grid of its own, and unknown values) leave the plan's
    choice unchanged.  Every value gives the oracle's result."""
    monkeypatch.setenv("ETIR_TILE", "7")
    monkeypatch.setenv("ETIR_DMA_VARIANT", variant)
    _, desc = run_case(torch_cuda, oracle, "zkm,zkn->zmn", dict(z=2, k=64, m=512, n=1024), dtype=eir.BF16,
                       seed=31)
    assert "bf16_dma_256x256" in desc, desc
    assert ("persistent" in desc) == persistent, desc


@pytest.mark.parametrize("phases,stagger", [("1", "0"), ("8", "2")])
def test_dma_persistent_stagger(torch_cuda, oracle, monkeypatch, phases, stagger):
    """Start stagger settings other than the default do not change results."""
    monkeypatch.setenv("ETIR_TILE", "7")
    monkeypatch.setenv("ETIR_DMA_PHASES", phases)
    monkeypatch.setenv("ETIR_DMA_STAGGER", stagger)
    _, desc = run_case(torch_cuda, oracle, "zkm,zkn->zmn", dict(z=2, k=64, m=512, n=1024), dtype=eir.BF16,
                       seed=29)
    assert "persistent" in desc, desc
