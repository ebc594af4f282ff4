"""GPU parity of the short-K panel kernel (tile "panel": K <= 64, one free
side of 65-256 kept in LDS, persistent workgroups streaming panels of the
long side).  Checker: the CPU oracle (fp64 accumulation) on the same seeded
inputs, output prefilled with random values (a store that is skipped shows);
fp32 relative Frobenius <= 1e-5."""
import numpy as np
import pytest

import einsum_ir_amd as eir
from tests.helpers import TOL_FP32, loops_for, parse_binary, rel_frobenius, tensor_numel
from tests.test_gpu_contract import run_case

pytestmark = pytest.mark.gpu

# shapes the planner gives the kernel by itself (at least 1024 panels: 64
# long-side rows each with a short side above 128, 128 rows up to 128)
DEFAULT_SHAPES = [
    # short kernel N (the output's unit-stride side), long operand K-contiguous:
    # the MERA root's kind (N = 243, K = 50), 256-wide short side
    ("mk,nk->mn", dict(m=70000, k=50, n=243)),
    # short kernel M, long operand unit-stride along the long side, odd K
    # (a zero k row), short side 65-128 (128-row panels)
    ("mk,kn->mn", dict(m=100, k=33, n=140000)),
    # K = 64 (every k row of LDS), short side a multiple of 32
    ("mk,nk->mn", dict(m=140000, k=64, n=128)),
    # long side split over two output dims (row offsets from the table):
    # out[a][n][j], kernel N = (a, j), short side 150
    ("ajk,nk->anj", dict(a=4, j=20000, k=40, n=150)),
    # K over two dims whose order differs between the operands (K offsets
    # from the tables), ragged last panel (L = 66667, moved back)
    ("mkl,nlk->mn", dict(m=66667, k=5, l=9, n=200)),
    # K = 1 (no K dim): an outer product
    ("m,n->mn", dict(m=140000, n=77)),
]


@pytest.mark.parametrize("expr,sizes", DEFAULT_SHAPES)
def test_panel_default(torch_cuda, oracle, monkeypatch, expr, sizes):
    monkeypatch.delenv("ETIR_TILE", raising=False)
    monkeypatch.delenv("ETIR_NO_PANEL", raising=False)
    _, desc = run_case(torch_cuda, oracle, expr, sizes, seed=sum(sizes.values()) % 1000)
    assert "panel" in desc, desc


# shapes with fewer panels than CUs, forced (ETIR_TILE=15): two panels, the
# second moved back to overlap the first; one panel per workgroup; both
# panel sizes
FORCED_SHAPES = [
    ("mk,nk->mn", dict(m=200, k=7, n=65)),
    ("mk,nk->mn", dict(m=3000, k=19, n=97)),
    ("km,kn->mn", dict(k=12, m=256, n=5000)),
    ("mk,nk->mn", dict(m=64 * 300 + 5, k=2, n=129)),
]


@pytest.mark.parametrize("expr,sizes", FORCED_SHAPES)
def test_panel_forced(torch_cuda, oracle, monkeypatch, expr, sizes):
    monkeypatch.setenv("ETIR_TILE", "15")
    _, desc = run_case(torch_cuda, oracle, expr, sizes, seed=7)
    assert "panel" in desc, desc


def test_panel_relu(torch_cuda, oracle):
    _, desc = run_case(torch_cuda, oracle, "mk,nk->mn", dict(m=70000, k=50, n=243), last=eir.RELU, seed=8)
    assert "panel" in desc, desc
    _, desc = run_case(torch_cuda, oracle, "mk,kn->mn", dict(m=100, k=33, n=140000), last=eir.RELU, seed=9)
    assert "panel" in desc, desc


@pytest.mark.parametrize("first,last", [(eir.UNDEFINED_KTYPE, eir.UNDEFINED_KTYPE), (eir.COPY, eir.UNDEFINED_KTYPE),
                                        (eir.ZERO, eir.ADD)])
def test_panel_other_touches_take_the_tiles(torch_cuda, oracle, first, last):
    """Accumulation into the output and aux tensors are not the panel
    kernel's: the planner keeps such nodes on the tiles (same results)."""
    _, desc = run_case(torch_cuda, oracle, "mk,nk->mn", dict(m=70000, k=50, n=243), first=first, last=last, seed=10)
    assert "panel" not in desc, desc


def test_panel_writes_nothing_past_the_output(torch_cuda, oracle):
    """Masked stores (short-side padding, rows past the last panel) go to an
    offset past the output's extent, which the buffer range check drops: a
    guard region after the output keeps its bit pattern."""
    torch = torch_cuda
    expr, sizes = "mk,nk->mn", dict(m=64 * 1030 + 17, k=9, n=200)
    left, right, out = parse_binary(expr)
    loops = loops_for(expr, sizes)
    rng = np.random.default_rng(11)
    a = rng.uniform(-1, 1, tensor_numel(left, sizes)).astype(np.float32)
    b = rng.uniform(-1, 1, tensor_numel(right, sizes)).astype(np.float32)
    n_out = tensor_numel(out, sizes)
    plan = eir.ContractionPlan(loops["dim_types"], loops["sizes"], loops["strides_left"],
                               loops["strides_right"], loops["strides_out"])
    assert "panel" in plan.describe(), plan.describe()
    guard = 64 * 1024
    buf = torch.full((n_out + guard,), float("nan"), device="cuda")
    plan.execute(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda(), buf, stream=torch.cuda.current_stream())
    torch.cuda.synchronize()
    plan.close()
    got = buf.cpu().numpy()
    assert np.isnan(got[n_out:]).all(), "a store landed past the output"
    ref = np.zeros(n_out, dtype=np.float32)
    oracle.contract(loops, a, b, ref)
    assert rel_frobenius(ref, got[:n_out]) <= TOL_FP32


def test_panel_switch_off(torch_cuda, oracle, monkeypatch):
    """ETIR_NO_PANEL leaves such shapes to the MFMA tiles (same results)."""
    monkeypatch.setenv("ETIR_NO_PANEL", "1")
    _, desc = run_case(torch_cuda, oracle, "mk,nk->mn", dict(m=70000, k=50, n=243), seed=12)
    assert "panel" not in desc, desc
