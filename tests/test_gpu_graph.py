"""GPU tests of EinsumExpression::eval_graph_async: one evaluation of the tree
recorded as a HIP graph and replayed.

The replays run the same kernels on the same data in the same order as eval(),
so every replay must reproduce eval()'s output bit for bit.  Between replays
the tests run eager work on the same and on other streams (eval(), torch fills)
and synchronise, and they check every replay, not only the first.  The small
expression is also checked against the path oracle (relative Frobenius error
<= 1e-5, fp32).
"""
import json
import os

import numpy as np
import pytest

import einsum_ir_amd as eir
from einsum_ir_amd import host
from tests.helpers import TOL_FP32, rel_frobenius, tensor_numel

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SMALL = ("iae,bf,dcba,cg,dh->hgfei", dict(a=2, b=3, c=4, d=5, e=6, f=7, g=8, h=9, i=10),
         [(1, 2), (0, 2), (0, 2), (0, 1)])


def _inputs(expr, sizes, seed, dist="uniform"):
    rng = np.random.default_rng(seed)
    ins = expr.split("->")[0].split(",")
    if dist == "uniform":
        return [rng.uniform(-1, 1, tensor_numel(t, sizes)).astype(np.float32) for t in ins]
    return [rng.standard_normal(tensor_numel(t, sizes)).astype(np.float32) / (1.0 if i == 0 else 45.25)
            for i, t in enumerate(ins)]


def _expression(torch, expr, sizes, path, arrays, stream):
    out = expr.split("->")[1]
    dev = [torch.from_numpy(a).cuda() for a in arrays]
    dout = torch.zeros(tensor_numel(out, sizes), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    e = host.Expression(expr, sizes, path, dev + [dout], dtype=eir.FP32, stream=stream)
    return e, dev, dout


def _check_replays(torch, e, dout, ref, replays=3):
    """Replays the graph several times with eager work in between; every
    replay must equal the eager result bit for bit."""
    for r in range(replays):
        dout.fill_(float("nan"))
        torch.cuda.synchronize()
        e.eval_graph()
        got = dout.cpu().numpy()
        assert np.array_equal(got, ref), f"replay {r} differs from eval()"
        # eager work between replays: an eager evaluation on the tree's stream
        e.eval()
        assert np.array_equal(dout.cpu().numpy(), ref)


def test_graph_small_expression(torch_cuda, oracle):
    torch = torch_cuda
    expr, sizes, path = SMALL
    arrays = _inputs(expr, sizes, 21)
    s = torch.cuda.Stream()
    e, dev, dout = _expression(torch, expr, sizes, path, arrays, s)
    e.eval()
    ref = dout.cpu().numpy()
    assert rel_frobenius(oracle.contract_path(expr, sizes, path, arrays), ref) <= TOL_FP32
    _check_replays(torch, e, dout, ref)
    e.close()


def test_graph_rerecorded_after_lock_changes(torch_cuda, oracle):
    """store_and_lock_data / unlock_data change what eval launches: the graph
    is recorded again and follows the new state."""
    torch = torch_cuda
    expr, sizes, path = SMALL
    arrays = _inputs(expr, sizes, 22)
    s = torch.cuda.Stream()
    e, dev, dout = _expression(torch, expr, sizes, path, arrays, s)
    ref = oracle.contract_path(expr, sizes, path, arrays)
    e.eval_graph()
    assert rel_frobenius(ref, dout.cpu().numpy()) <= TOL_FP32
    e.store_and_lock_data(3)
    dev[3].zero_()                      # the locked copy is used, not this buffer
    torch.cuda.synchronize()
    for _ in range(2):
        dout.zero_()
        torch.cuda.synchronize()
        e.eval_graph()
        assert rel_frobenius(ref, dout.cpu().numpy()) <= TOL_FP32
    e.unlock_data(3)                    # back to the (now zero) external buffer
    dout.fill_(1.0)
    torch.cuda.synchronize()
    e.eval_graph()
    assert not np.any(dout.cpu().numpy())
    e.close()


def test_graph_needs_a_stream(torch_cuda):
    torch = torch_cuda
    expr, sizes, path = SMALL
    e, dev, dout = _expression(torch, expr, sizes, path, _inputs(expr, sizes, 23), None)
    with pytest.raises(eir.EinsumIrError) as err:
        e.eval_graph()
    assert err.value.code == eir.UNDEFINED_ERROR
    e.eval()                            # the eager path is unaffected
    e.close()


def test_graph_c4_mlp_tree_full_size(torch_cuda):
    """BASELINE config 4 (four 4096x2048x2048 fp32 contractions) replayed."""
    torch = torch_cuda
    b, w = 4096, 2048
    expr = "bi,ih,hj,jk,ko->bo"
    sizes = dict(b=b, i=w, h=w, j=w, k=w, o=w)
    arrays = _inputs(expr, sizes, 4, dist="normal")
    s = torch.cuda.Stream()
    e, dev, dout = _expression(torch, expr, sizes, [(0, 1), (0, 3), (0, 2), (0, 1)], arrays, s)
    e.eval()
    ref = dout.cpu().numpy()
    assert np.isfinite(ref).all() and np.any(ref)
    _check_replays(torch, e, dout, ref, replays=2)
    e.close()


def test_graph_c5_network_full_size(torch_cuda):
    """BASELINE config 5 (nine contractions, split-K reductions, permutes) replayed."""
    torch = torch_cuda
    fx = json.load(open(os.path.join(ROOT, "tests", "golden", "c5_network.json")))
    expr, sizes, path = fx["expr"], fx["sizes"], [tuple(p) for p in fx["path"]]
    arrays = _inputs(expr, sizes, fx["seed"])
    s = torch.cuda.Stream()
    e, dev, dout = _expression(torch, expr, sizes, path, arrays, s)
    e.eval()
    ref = dout.cpu().numpy()
    assert np.isfinite(ref).all() and np.any(ref)
    _check_replays(torch, e, dout, ref, replays=2)
    e.close()
