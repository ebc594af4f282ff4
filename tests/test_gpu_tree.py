"""GPU parity of the operator classes and the device-resident tree path
(libeinsum_ir.so: BinaryContractionHip, UnaryHip, EinsumExpression, EinsumTree).

Mirrors the reference's tree tests (reference src/backend/EinsumNode.test.torch.cpp,
src/frontend/EinsumExpression.test.torch.cpp, src/frontend/EinsumTree.test.torch.cpp)
with seeded inputs.  Checkers: the path oracle (oracle_contract per node) at
sizes it finishes in seconds; at the BASELINE config-4/5 sizes numpy.einsum in
float64 along the same path (the library routine the oracle is pinned to).
Bar: relative Frobenius error <= 1e-5 (fp32).
"""
import json
import os

import numpy as np
import pytest

import einsum_ir_amd as eir
from einsum_ir_amd import host
from tests.helpers import TOL_FP32, TOL_BF16, rel_frobenius, tensor_numel

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _dev(torch, x):
    if x.dtype == np.uint16:
        return torch.from_numpy(x.view(np.int16)).cuda()
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def _run_expression(torch, expr, sizes, path, arrays, lock=()):
    ins, out = expr.split("->")
    dev = [_dev(torch, a) for a in arrays]
    dout = torch.zeros(tensor_numel(out, sizes), dtype=torch.float32, device="cuda")
    e = host.Expression(expr, sizes, path, dev + [dout], dtype=eir.FP32)
    for t in lock:
        e.store_and_lock_data(t)
    e.eval()
    got = dout.cpu().numpy()
    return e, got


EXPRESSIONS = [
    # (expression, sizes, path) -- shapes of the reference's expression/tree tests
    ("da,dce,bec->abc", dict(a=3, b=4, c=5, d=6, e=7), [(1, 2), (0, 1)]),
    ("iae,bf,dcba,cg,dh->hgfei", dict(a=2, b=3, c=4, d=5, e=6, f=7, g=8, h=9, i=10),
     [(1, 2), (0, 2), (0, 2), (0, 1)]),
    ("bi,ih,hj->bj", dict(b=96, i=80, h=72, j=64), [(0, 1), (0, 1)]),
    ("abcd,cdef,efgh->abgh", dict(a=4, b=5, c=6, d=7, e=3, f=4, g=5, h=6), [(0, 1), (0, 1)]),
    ("xab,ybc,zcd->xyzad", dict(x=2, y=3, z=2, a=16, b=8, c=12, d=10), [(0, 1), (0, 1)]),
]


@pytest.mark.parametrize("expr,sizes,path", EXPRESSIONS)
def test_expression_matches_path_oracle(torch_cuda, oracle, expr, sizes, path):
    rng = np.random.default_rng(sum(map(ord, expr)))
    ins = expr.split("->")[0].split(",")
    arrays = [rng.uniform(-1, 1, tensor_numel(t, sizes)).astype(np.float32) for t in ins]
    e, got = _run_expression(torch_cuda, expr, sizes, path, arrays)
    ref = oracle.contract_path(expr, sizes, path, arrays)
    assert rel_frobenius(ref, got) <= TOL_FP32
    # num_ops: sum over nodes of 2*C*M*N*K minus C*M*N for the ZERO first touch
    assert e.num_ops() > 0
    e.close()


def test_expression_locked_inputs(torch_cuda, oracle):
    """store_and_lock_data: inputs are copied (and permuted) once; later changes
    of the external buffers are ignored (reference EinsumNode.cpp:458-479)."""
    torch = torch_cuda
    expr, sizes, path = EXPRESSIONS[1]
    rng = np.random.default_rng(3)
    ins = expr.split("->")[0].split(",")
    arrays = [rng.uniform(-1, 1, tensor_numel(t, sizes)).astype(np.float32) for t in ins]
    dev = [_dev(torch, a) for a in arrays]
    dout = torch.zeros(tensor_numel("hgfei", sizes), dtype=torch.float32, device="cuda")
    e = host.Expression(expr, sizes, path, dev + [dout])
    e.store_and_lock_data(2)
    e.store_and_lock_data(0)
    dev[2].zero_()
    dev[0].zero_()
    e.eval()
    ref = oracle.contract_path(expr, sizes, path, arrays)
    assert rel_frobenius(ref, dout.cpu().numpy()) <= TOL_FP32
    e.unlock_data(2)
    e.unlock_data(0)
    e.eval()
    assert not np.any(dout.cpu().numpy())
    with pytest.raises(eir.EinsumIrError) as err:
        e.store_and_lock_data(7)
    assert err.value.code == eir.INVALID_ID
    e.close()


def test_c4_mlp_tree_full_size(torch_cuda):
    """bi,ih,hj,jk,ko->bo, b=4096, widths 2048, fp32, left-to-right path."""
    torch = torch_cuda
    b, w = 4096, 2048
    sizes = dict(b=b, i=w, h=w, j=w, k=w, o=w)
    rng = np.random.default_rng(4)
    x = rng.standard_normal(b * w).astype(np.float32)
    ws = [(rng.standard_normal(w * w) / np.sqrt(w)).astype(np.float32) for _ in range(4)]
    e, got = _run_expression(torch, "bi,ih,hj,jk,ko->bo", sizes, [(0, 1), (0, 3), (0, 2), (0, 1)], [x] + ws)
    assert e.num_ops() == 4 * (2 * b * w * w - b * w)
    ref = x.astype(np.float64).reshape(b, w)
    for wm in ws:
        ref = ref @ wm.astype(np.float64).reshape(w, w)
    assert rel_frobenius(ref, got) <= TOL_FP32
    e.close()


def test_c5_tensor_network_full_size(torch_cuda):
    """the committed random tensor network (~50 GFLOP)."""
    torch = torch_cuda
    fx = json.load(open(os.path.join(ROOT, "tests", "golden", "c5_network.json")))
    expr, sizes, path = fx["expr"], fx["sizes"], [tuple(p) for p in fx["path"]]
    ins, out = expr.split("->")
    ins = ins.split(",")
    rng = np.random.default_rng(fx["seed"])
    arrays = [rng.uniform(-1, 1, tensor_numel(t, sizes)).astype(np.float32) for t in ins]
    e, got = _run_expression(torch, expr, sizes, path, arrays)
    ops = [a.astype(np.float64).reshape([sizes[d] for d in t]) for a, t in zip(arrays, ins)]
    ref = np.einsum(expr, *ops, optimize=["einsum_path"] + [tuple(p) for p in path])
    assert rel_frobenius(ref, got) <= TOL_FP32
    e.close()


def test_c5_scaled_against_path_oracle(torch_cuda, oracle):
    """The config-5 network with every mode of size 2: checked by the path oracle."""
    fx = json.load(open(os.path.join(ROOT, "tests", "golden", "c5_network.json")))
    expr, path = fx["expr"], [tuple(p) for p in fx["path"]]
    sizes = {k: 2 for k in fx["sizes"]}
    ins = expr.split("->")[0].split(",")
    rng = np.random.default_rng(55)
    arrays = [rng.uniform(-1, 1, tensor_numel(t, sizes)).astype(np.float32) for t in ins]
    e, got = _run_expression(torch_cuda, expr, sizes, path, arrays)
    ref = oracle.contract_path(expr, sizes, path, arrays)
    assert rel_frobenius(ref, got) <= TOL_FP32
    e.close()


def test_tree_format_with_unary_node(torch_cuda, oracle):
    """bench_tree's example: a unary permutation node and two binary nodes."""
    torch = torch_cuda
    tree = "[[3,0]->[0,3]],[[3,2,4],[1,4,2]->[1,2,3]]->[0,1,2]"
    sizes = [2, 3, 4, 5, 6]
    assert host.Tree.count_nodes(tree) == 6
    rng = np.random.default_rng(6)
    n = lambda ids: int(np.prod([sizes[i] for i in ids]))
    t30 = rng.uniform(-1, 1, n([3, 0])).astype(np.float32)
    t324 = rng.uniform(-1, 1, n([3, 2, 4])).astype(np.float32)
    t142 = rng.uniform(-1, 1, n([1, 4, 2])).astype(np.float32)
    out = torch.zeros(n([0, 1, 2]), device="cuda")
    tensors = [_dev(torch, t30), None, _dev(torch, t324), _dev(torch, t142), None, out]
    tr = host.Tree(tree, sizes, tensors)
    tr.eval()
    A = t30.astype(np.float64).reshape(5, 2)                  # [3,0]
    B = t324.astype(np.float64).reshape(5, 4, 6)              # [3,2,4]
    Cc = t142.astype(np.float64).reshape(3, 6, 4)             # [1,4,2]
    T = np.einsum("dce,bec->bcd", B, Cc)                      # [1,2,3]
    ref = np.einsum("da,bcd->abc", A, T)                      # [0,1,2]
    assert rel_frobenius(ref, out.cpu().numpy()) <= TOL_FP32
    tr.close()


def test_binary_contraction_class(torch_cuda, oracle):
    """BinaryContractionHip through the 18-argument init: BASELINE config 1 + num_ops."""
    torch = torch_cuda
    sizes = dict(a=32, b=16, c=32, d=16, k=32, l=16)
    bc = host.Binary("abkl,cdkl->abcd", sizes)
    nd, sz = bc.sizes_cmnk()
    assert nd == [0, 2, 2, 2] and sz == [1, 512, 512, 512]
    assert bc.num_ops() == 2 * 512 ** 3 - 512 * 512
    rng = np.random.default_rng(1)
    a = rng.uniform(-1, 1, 512 * 512).astype(np.float32)
    b = rng.uniform(-1, 1, 512 * 512).astype(np.float32)
    out = torch.empty(512 * 512, device="cuda")
    bc.contract(_dev(torch, a), _dev(torch, b), out)
    ref = a.astype(np.float64).reshape(512, 512) @ b.astype(np.float64).reshape(512, 512).T
    assert rel_frobenius(ref, out.cpu().numpy()) <= TOL_FP32
    bc.close()


@pytest.mark.parametrize("bcast", ["row", "col", "scalar", "full"])
def test_binary_copy_relu_with_aux_outer_sizes(torch_cuda, oracle, bcast):
    """Bias COPY (broadcast through aux outer sizes of 1) + RELU last touch
    (reference BinaryContractionTpp.test.torch.cpp:77-367, 725-824)."""
    torch = torch_cuda
    sizes = dict(m=40, k=24, n=48)
    aux_outer = {"row": dict(m=1, k=24, n=48), "col": dict(m=40, k=24, n=1),
                 "scalar": dict(m=1, k=24, n=1), "full": dict(m=40, k=24, n=48)}[bcast]
    bc = host.Binary("mk,kn->mn", sizes, ktype_first_touch=eir.COPY, ktype_last_touch=eir.RELU,
                     aux_outer_sizes=aux_outer)
    rng = np.random.default_rng(9)
    a = rng.uniform(-1, 1, 40 * 24).astype(np.float32)
    b = rng.uniform(-1, 1, 24 * 48).astype(np.float32)
    x = rng.uniform(-1, 1, aux_outer["m"] * aux_outer["n"]).astype(np.float32)
    out = torch.empty(40 * 48, device="cuda")
    bc.contract(_dev(torch, a), _dev(torch, b), out, aux=_dev(torch, x))
    ref = a.astype(np.float64).reshape(40, 24) @ b.astype(np.float64).reshape(24, 48)
    ref = np.maximum(ref + x.astype(np.float64).reshape(aux_outer["m"], aux_outer["n"]), 0.0)
    assert rel_frobenius(ref, out.cpu().numpy()) <= TOL_FP32
    bc.close()


def test_binary_bf16(torch_cuda, oracle):
    torch = torch_cuda
    sizes = dict(z=2, a=4, m=64, b=4, n=64, k=256)
    bc = host.Binary("zakm,zbkn->zabmn", sizes, dtype_left=eir.BF16, dtype_right=eir.BF16)
    rng = np.random.default_rng(2)
    a = oracle.f32_to_bf16(rng.uniform(-1, 1, 2 * 4 * 256 * 64).astype(np.float32))
    b = oracle.f32_to_bf16(rng.uniform(-1, 1, 2 * 4 * 256 * 64).astype(np.float32))
    out = torch.empty(2 * 4 * 4 * 64 * 64, device="cuda")
    bc.contract(_dev(torch, a), _dev(torch, b), out)
    loops = eir.binary_loops("zakm,zbkn->zabmn", sizes)
    ref = np.zeros(out.numel(), dtype=np.float32)
    oracle.contract(loops, a, b, ref, dtype_left=oracle.BF16, dtype_right=oracle.BF16)
    assert rel_frobenius(ref, out.cpu().numpy()) <= TOL_BF16
    bc.close()


def test_unary_class_c2(torch_cuda, oracle):
    """UnaryHip through Unary::init: BASELINE config 2, bit-exact."""
    torch = torch_cuda
    u = host.Unary("abcd->dbca", dict(a=64, b=64, c=64, d=64))
    rng = np.random.default_rng(2)
    x = rng.uniform(-1, 1, 64 ** 4).astype(np.float32)
    out = torch.empty(64 ** 4, device="cuda")
    u.eval(_dev(torch, x), out)
    ref = np.transpose(x.reshape(64, 64, 64, 64), (3, 1, 2, 0)).ravel()
    np.testing.assert_array_equal(out.cpu().numpy(), ref)
    u.close()


def test_unsupported_backend_is_reported(torch_cuda, monkeypatch):
    """EINSUM_IR_BACKEND naming a CPU backend of the reference: INVALID_BACKEND."""
    torch = torch_cuda
    monkeypatch.setenv("EINSUM_IR_BACKEND", "TPP")
    dev = [torch.zeros(4, device="cuda") for _ in range(3)]
    with pytest.raises(eir.EinsumIrError) as err:
        host.Expression("ab,bc->ac", dict(a=2, b=2, c=2), [(0, 1)], dev)
    assert err.value.code == eir.INVALID_BACKEND


@pytest.mark.parametrize("idx", [1, 3, 4])
def test_expression_bf16(torch_cuda, oracle, idx):
    """A bf16 tree: bf16 inputs, intermediates and output (RNE), fp32
    accumulation in every node.  Checker: the path oracle with every step's
    result rounded to bf16 on the same bf16-rounded inputs; bar 2e-3 relative
    Frobenius (fp32 against fp64 accumulation can move a rounding by one bf16
    step)."""
    torch = torch_cuda
    expr, sizes, path = EXPRESSIONS[idx]
    rng = np.random.default_rng(40 + idx)
    ins = expr.split("->")[0].split(",")
    out = expr.split("->")[1]
    arrays = [oracle.f32_to_bf16(rng.uniform(-1, 1, tensor_numel(t, sizes)).astype(np.float32)) for t in ins]
    dev = [_dev(torch, a) for a in arrays]
    dout = torch.zeros(tensor_numel(out, sizes), dtype=torch.int16, device="cuda")
    e = host.Expression(expr, sizes, path, dev + [dout], dtype=eir.BF16)
    e.eval()
    got = oracle.bf16_to_f32(dout.cpu().numpy().view(np.uint16))
    ref = oracle.contract_path(expr, sizes, path, [oracle.bf16_to_f32(a) for a in arrays], round_bf16=True)
    assert rel_frobenius(ref, got) <= TOL_BF16
    e.close()
