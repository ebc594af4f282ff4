"""GPU parity of the one-short-side kernel (tile "skinny": kernel M or N of 2
to 64, one thread per index of the long side).  Checker: the CPU oracle (fp64
accumulation) on the same seeded inputs; fp32 relative Frobenius <= 1e-5,
bf16 inputs or output <= 2e-3."""
import numpy as np
import pytest

import einsum_ir_amd as eir
from tests.helpers import TOL_FP32, loops_for, parse_binary, rel_frobenius, tensor_numel
from tests.test_gpu_contract import run_case

pytestmark = pytest.mark.gpu

# shapes the planner gives the kernel by itself
DEFAULT_SHAPES = [
    # short M, long operand K-contiguous: 16-byte vectors along K
    ("mk,nk->mn", dict(m=11, k=24, n=70000), "kvec"),
    # short N (the output's unit-stride side), long operand A K-contiguous
    ("mk,nk->mn", dict(m=70000, k=40, n=9), "kvec"),
    # long operand unit-stride along the long side: coalesced scalar loads
    ("km,kn->mn", dict(k=11, m=5, n=80000), ""),
    # short side 45 with K <= 64, the MERA shape
    ("mk,kn->mn", dict(m=45, k=11, n=70000), ""),
    # short sides of 33-48 (SMAX 48: the staging's short indices repeat
    # every 3 elements of a thread), K over two chunks
    ("km,kn->mn", dict(k=40, m=33, n=70000), ""),
    ("mk,nk->mn", dict(m=70000, k=52, n=48), "kvec"),
    # K over several 32-k chunks with a tail, K % 4 != 0: no vectors
    ("mk,nk->mn", dict(m=16, k=102, n=70000), ""),
    # a C dim (grid rows)
    ("zmk,znk->zmn", dict(z=3, m=10, k=20, n=90000), "kvec"),
    # two K dims in different orders: K offsets from the table
    ("mlk,nkl->mn", dict(m=12, k=5, l=6, n=70000), ""),
]


@pytest.mark.parametrize("expr,sizes,flag", DEFAULT_SHAPES)
def test_skinny_default(torch_cuda, oracle, monkeypatch, expr, sizes, flag):
    monkeypatch.delenv("ETIR_TILE", raising=False)
    _, desc = run_case(torch_cuda, oracle, expr, sizes, seed=sum(sizes.values()) % 1000)
    assert "skinny" in desc, desc
    assert (" kvec" in desc) == (flag == "kvec"), desc


# shapes the planner leaves to the MFMA tiles, forced (ETIR_TILE=14): short
# sides from 2 to 64, K up to several chunks, every SMAX instantiation
FORCED_SHAPES = [
    ("mk,nk->mn", dict(m=2, k=7, n=3000)),
    ("mk,kn->mn", dict(m=30, k=300, n=1000)),
    ("km,nk->mn", dict(k=65, m=64, n=2000)),
    ("mk,nk->mn", dict(m=1500, k=33, n=24)),
]


@pytest.mark.parametrize("expr,sizes", FORCED_SHAPES)
def test_skinny_forced(torch_cuda, oracle, monkeypatch, expr, sizes):
    monkeypatch.setenv("ETIR_TILE", "14")
    _, desc = run_case(torch_cuda, oracle, expr, sizes, seed=7)
    assert "skinny" in desc, desc


@pytest.mark.parametrize("first,last", [(eir.COPY, eir.RELU), (eir.ADD, eir.UNDEFINED_KTYPE),
                                        (eir.UNDEFINED_KTYPE, eir.ADD), (eir.ZERO, eir.RELU)])
def test_skinny_touch_kernels(torch_cuda, oracle, first, last):
    _, desc = run_case(torch_cuda, oracle, "mk,nk->mn", dict(m=11, k=24, n=70000), first=first, last=last,
                       seed=first + 5 * last)
    assert "skinny" in desc, desc


def test_skinny_bf16(torch_cuda, oracle):
    _, desc = run_case(torch_cuda, oracle, "mk,nk->mn", dict(m=11, k=24, n=70000), dtype=eir.BF16, seed=3)
    assert "skinny" in desc and "kvec" in desc, desc
    _, desc = run_case(torch_cuda, oracle, "km,kn->mn", dict(k=11, m=5, n=80000), dtype=eir.BF16,
                       dtype_out=eir.BF16, seed=4)
    assert "skinny" in desc, desc


def test_skinny_misaligned_long_operand(torch_cuda, oracle):
    """The long operand one element off a 16-byte boundary: the launch reads
    it element by element instead of in vectors, same result as aligned."""
    torch = torch_cuda
    expr, sizes = "mk,nk->mn", dict(m=11, k=24, n=70000)
    left, right, out = parse_binary(expr)
    loops = loops_for(expr, sizes)
    rng = np.random.default_rng(9)
    a = rng.uniform(-1, 1, tensor_numel(left, sizes)).astype(np.float32)
    b = rng.uniform(-1, 1, tensor_numel(right, sizes)).astype(np.float32)
    plan = eir.ContractionPlan(loops["dim_types"], loops["sizes"], loops["strides_left"],
                               loops["strides_right"], loops["strides_out"])
    desc = plan.describe()
    assert "skinny" in desc and "kvec" in desc, desc
    da = torch.from_numpy(a).cuda()
    buf_b = torch.zeros(b.size + 1, device="cuda")
    buf_b[1:] = torch.from_numpy(b).cuda()
    db_al = torch.from_numpy(b).cuda()
    o_mis = torch.zeros(tensor_numel(out, sizes), device="cuda")
    o_al = torch.zeros_like(o_mis)
    s = torch.cuda.current_stream()
    plan.execute(da, buf_b[1:], o_mis, stream=s)
    plan.execute(da, db_al, o_al, stream=s)
    torch.cuda.synchronize()
    plan.close()
    assert torch.equal(o_mis, o_al), "vector and element loads sum differently"
    ref = np.zeros(tensor_numel(out, sizes), dtype=np.float32)
    oracle.contract(loops, a, b, ref)
    assert rel_frobenius(ref, o_al.cpu().numpy()) <= TOL_FP32


def test_skinny_switch_off(torch_cuda, oracle, monkeypatch):
    """ETIR_NO_SKINNY leaves such shapes to the MFMA tiles (same results)."""
    monkeypatch.setenv("ETIR_NO_SKINNY", "1")
    _, desc = run_case(torch_cuda, oracle, "mk,nk->mn", dict(m=11, k=24, n=70000), seed=12)
    assert "skinny" not in desc, desc


# outputs laid out as [long][short] with the short side unit-stride: the
# workgroup writes its outputs as one block through LDS (" blk")
BLOCK_SHAPES = [
    # short kernel N of 9 (one chunk of 9), long operand in K vectors
    ("mk,nk->mn", dict(m=70000, k=40, n=9)),
    # short kernel M of 45 (SMAX 64: chunks of 16, 16, 13), output [n][m]
    ("mk,kn->nm", dict(m=45, k=11, n=70000)),
    # a C dim: one block per workgroup per C index
    ("zmk,znk->zmn", dict(z=3, m=30000, k=6, n=12)),
    # short side over two output dims, ragged last workgroup (70001 rows)
    ("mk,kst->mst", dict(m=70001, k=5, s=4, t=5)),
    # short side 64 (four full chunks)
    ("mk,nk->mn", dict(m=70000, k=20, n=64)),
]


@pytest.mark.parametrize("expr,sizes", BLOCK_SHAPES)
def test_skinny_block_store(torch_cuda, oracle, monkeypatch, expr, sizes):
    monkeypatch.delenv("ETIR_TILE", raising=False)
    _, desc = run_case(torch_cuda, oracle, expr, sizes, seed=sum(sizes.values()) % 1000)
    assert "skinny" in desc and " blk" in desc, desc


def test_skinny_block_store_relu_bf16(torch_cuda, oracle):
    _, desc = run_case(torch_cuda, oracle, "mk,kn->nm", dict(m=45, k=11, n=70000), last=eir.RELU, seed=21)
    assert " blk" in desc, desc
    _, desc = run_case(torch_cuda, oracle, "mk,kn->nm", dict(m=45, k=11, n=70000), dtype=eir.BF16,
                       dtype_out=eir.BF16, seed=22)
    assert " blk" in desc, desc


def test_skinny_block_store_only_for_its_layout(torch_cuda, oracle):
    """Accumulation into the output reads it per element, and a short side
    that is not the output's unit-stride run (the MERA chain's
    [long / 10][short][long % 10]) has no block: the planner keeps the
    per-thread stores there (same results)."""
    _, desc = run_case(torch_cuda, oracle, "mk,kn->nm", dict(m=45, k=11, n=70000), first=eir.ADD, seed=23)
    assert "skinny" in desc and " blk" not in desc, desc
    _, desc = run_case(torch_cuda, oracle, "akr,ks->asr", dict(a=7000, k=11, r=10, s=45), seed=25)
    assert "skinny" in desc and " blk" not in desc, desc


def test_skinny_block_store_writes_nothing_past_the_output(torch_cuda, oracle):
    """The last workgroup's block ends with the output: a guard region after
    the output keeps its bit pattern."""
    torch = torch_cuda
    expr, sizes = "mk,nk->mn", dict(m=64 * 1030 + 17, k=9, n=13)
    left, right, out = parse_binary(expr)
    loops = loops_for(expr, sizes)
    rng = np.random.default_rng(24)
    a = rng.uniform(-1, 1, tensor_numel(left, sizes)).astype(np.float32)
    b = rng.uniform(-1, 1, tensor_numel(right, sizes)).astype(np.float32)
    n_out = tensor_numel(out, sizes)
    plan = eir.ContractionPlan(loops["dim_types"], loops["sizes"], loops["strides_left"],
                               loops["strides_right"], loops["strides_out"])
    assert " blk" in plan.describe(), plan.describe()
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
