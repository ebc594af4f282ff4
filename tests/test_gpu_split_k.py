"""GPU parity of split-K contractions: few output tiles and a long K make the
planner run the contraction as a partial contraction (outer K loops turned
into batch loops writing workspace slices) plus a reduction that applies the
touch kernels.  Checker: the CPU oracle (fp64 accumulation); fp32 relative
Frobenius <= 1e-5, bf16 inputs <= 2e-3."""
import numpy as np
import pytest

import einsum_ir_amd as eir
from tests.test_gpu_contract import run_case

pytestmark = pytest.mark.gpu


def _split_of(desc):
    return int(desc.split("split-K S=")[1].split()[0]) if "split-K" in desc else 1


@pytest.mark.parametrize("first,last", [(eir.ZERO, eir.UNDEFINED_KTYPE), (eir.COPY, eir.UNDEFINED_KTYPE),
                                        (eir.ADD, eir.UNDEFINED_KTYPE), (eir.UNDEFINED_KTYPE, eir.UNDEFINED_KTYPE),
                                        (eir.ZERO, eir.RELU), (eir.COPY, eir.RELU), (eir.ZERO, eir.ADD)])
def test_split_touch_kernels(torch_cuda, oracle, first, last):
    _, desc = run_case(torch_cuda, oracle, "mk,kn->mn", dict(m=64, k=4096, n=96), first=first, last=last)
    assert _split_of(desc) > 1, desc
    # a dense output (with an aux tensor of its own layout) is reduced as
    # flat arrays
    assert "reduce flat" in desc, desc


@pytest.mark.parametrize("aux_outer,flat", [
    # a bias over n, broadcast over the outermost dim m: aux offset o % n
    (dict(m=1, n=96), True),
    # broadcast over the innermost dim n: the table reduction
    (dict(m=64, n=1), False),
])
@pytest.mark.parametrize("first,last", [(eir.COPY, eir.RELU), (eir.ZERO, eir.ADD), (eir.ADD, eir.UNDEFINED_KTYPE)])
def test_split_broadcast_aux(torch_cuda, oracle, aux_outer, flat, first, last):
    _, desc = run_case(torch_cuda, oracle, "mk,kn->mn", dict(m=64, k=4096, n=96), first=first, last=last,
                       aux_outer=aux_outer, seed=64)
    assert _split_of(desc) > 1, desc
    assert ("reduce flat" in desc) == flat, desc


@pytest.mark.parametrize("expr,sizes", [
    # 6111 outputs: the last thread of the 4-wide flat reduction holds 3
    ("mk,kn->mn", dict(m=63, k=4096, n=97)),
    # the output's dims in another order than the kernel's M and N (dense all
    # the same: the flat reduction does not need the element order)
    ("akb,kn->nab", dict(a=7, k=4096, b=9, n=33)),
])
def test_split_flat_reduction(torch_cuda, oracle, expr, sizes):
    _, desc = run_case(torch_cuda, oracle, expr, sizes, seed=61)
    assert _split_of(desc) > 1 and "reduce flat" in desc, desc
    _, desc = run_case(torch_cuda, oracle, expr, sizes, last=eir.RELU, seed=62)
    assert "reduce flat" in desc, desc


def test_split_padded_output_takes_the_table_reduction(torch_cuda, oracle):
    """An output with a gap between its rows is not dense: the reduction
    walks the offset tables (and leaves the gap alone); the values agree with
    the flat reduction of the same contraction into a dense output."""
    torch = torch_cuda
    from tests.helpers import loops_for
    m, k, n, pad = 64, 4096, 96, 5
    loops = loops_for("mk,kn->mn", dict(m=m, k=k, n=n))
    rng = np.random.default_rng(63)
    a = torch.from_numpy(rng.uniform(-1, 1, m * k).astype(np.float32)).cuda()
    b = torch.from_numpy(rng.uniform(-1, 1, k * n).astype(np.float32)).cuda()
    outs = {}
    for row in (n, n + pad):
        strides_out = list(loops["strides_out"])
        for i, s_ in enumerate(strides_out):
            if s_ == n:
                strides_out[i] = row
        plan = eir.ContractionPlan(loops["dim_types"], loops["sizes"], loops["strides_left"],
                                   loops["strides_right"], strides_out)
        desc = plan.describe()
        buf = torch.full((m * row,), float("nan"), device="cuda")
        plan.execute(a, b, buf, stream=torch.cuda.current_stream())
        torch.cuda.synchronize()
        plan.close()
        assert _split_of(desc) > 1, desc
        assert ("reduce flat" in desc) == (row == n), desc
        got = buf.cpu().numpy().reshape(m, row)
        if row > n:
            assert np.isnan(got[:, n:]).all(), "the reduction wrote into the gap"
        outs[row] = got[:, :n]
    ref = np.zeros(m * n, dtype=np.float32)
    oracle.contract(loops, a.cpu().numpy(), b.cpu().numpy(), ref)
    for got in outs.values():
        assert np.linalg.norm(got.ravel() - ref) / np.linalg.norm(ref) <= 1e-5
    assert np.linalg.norm(outs[n] - outs[n + pad]) / np.linalg.norm(outs[n]) <= 1e-6


def test_split_bf16_inputs_and_output(torch_cuda, oracle):
    _, desc = run_case(torch_cuda, oracle, "km,nk->mn", dict(k=2048, m=96, n=64), dtype=eir.BF16,
                       dtype_out=eir.BF16)
    assert _split_of(desc) > 1 and "reduce flat" in desc, desc


def test_split_multi_loop_k(torch_cuda, oracle):
    """K spread over several non-adjacent loops (table K), factored split."""
    _, desc = run_case(torch_cuda, oracle, "akbmc,bcknd->amnd", dict(a=2, k=16, b=12, m=8, c=10, n=8, d=4))
    assert _split_of(desc) > 1, desc


def test_split_c5_node_shape(torch_cuda, oracle):
    """The shape of the costliest node of BASELINE config 5 (M=64, N=1024,
    K=32768 over six loops), scaled down in K so the oracle stays fast."""
    sizes = dict(a=8, b=8, c=8, d=8, e=16, p=2, q=2, r=4, s=8, t=4)
    _, desc = run_case(torch_cuda, oracle, "pqrstab,pqrstecd->abecd", sizes, seed=55)
    assert _split_of(desc) > 1, desc


def test_split_matches_unsplit(torch_cuda, oracle, monkeypatch):
    """Same inputs through the split and the unsplit plan."""
    got_s, desc_s = run_case(torch_cuda, oracle, "mk,kn->mn", dict(m=128, k=8192, n=64), seed=9)
    monkeypatch.setenv("ETIR_NO_SPLIT_K", "1")
    got_u, desc_u = run_case(torch_cuda, oracle, "mk,kn->mn", dict(m=128, k=8192, n=64), seed=9)
    assert _split_of(desc_s) > 1 and _split_of(desc_u) == 1, (desc_s, desc_u)
    err = np.linalg.norm(got_s - got_u) / np.linalg.norm(got_u)
    assert err <= 1e-5
