"""Host tensors through the synchronous operator calls.

The reference's callers pass host memory (at::Tensor CPU data, reference
src/bench_binary.cpp:132-134).  BinaryContractionHip::contract,
UnaryHip::eval, EinsumNode::eval and store_and_lock_data stage such tensors
through device copies (csrc/host/backend/HostStaging.h); the results must
equal those of the same call on device tensors bit for bit (the same kernels
run on the same values), and a recorded graph must refuse host tensors.
"""
import ctypes

import numpy as np
import pytest

import einsum_ir_amd as eir
from einsum_ir_amd import host
from einsum_ir_amd._lib import hip_lib
from tests.helpers import TOL_FP32, rel_frobenius

pytestmark = pytest.mark.gpu


def _hp(a):
    """Address of a numpy array (pageable host memory)."""
    return a.ctypes.data


def test_pointer_kinds(torch_cuda):
    torch = torch_cuda
    lib = hip_lib()
    d = torch.zeros(16, device="cuda")
    h = np.zeros(16, dtype=np.float32)
    p = torch.zeros(16).pin_memory()
    assert lib.etir_hip_pointer_is_device(ctypes.c_void_p(d.data_ptr())) == 1
    assert lib.etir_hip_pointer_is_device(ctypes.c_void_p(d.data_ptr() + 4)) == 1
    assert lib.etir_hip_pointer_is_device(ctypes.c_void_p(_hp(h))) == 0
    assert lib.etir_hip_pointer_is_device(ctypes.c_void_p(p.data_ptr())) == 1
    assert lib.etir_hip_pointer_is_device(None) == 0


@pytest.mark.parametrize("where", ["left", "right", "out", "all"])
def test_binary_host_tensors(torch_cuda, where):
    torch = torch_cuda
    sizes = dict(a=8, b=6, c=10, d=4, k=12, l=5)
    bc = host.Binary("abkl,cdkl->abcd", sizes)
    rng = np.random.default_rng(1)
    a = rng.uniform(-1, 1, 8 * 6 * 12 * 5).astype(np.float32)
    b = rng.uniform(-1, 1, 10 * 4 * 12 * 5).astype(np.float32)
    ref = torch.empty(8 * 6 * 10 * 4, device="cuda")
    bc.contract(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda(), ref)
    out_h = np.full(8 * 6 * 10 * 4, np.nan, dtype=np.float32)
    out_d = torch.empty(8 * 6 * 10 * 4, device="cuda")
    args_l = _hp(a) if where in ("left", "all") else torch.from_numpy(a).cuda()
    args_r = _hp(b) if where in ("right", "all") else torch.from_numpy(b).cuda()
    args_o = _hp(out_h) if where in ("out", "all") else out_d
    bc.contract(args_l, args_r, args_o)
    got = out_h if where in ("out", "all") else out_d.cpu().numpy()
    assert np.array_equal(got, ref.cpu().numpy())
    bc.close()


def test_binary_host_aux_and_accumulate(torch_cuda):
    """Bias COPY from a host aux tensor, and a host output read back for ADD."""
    torch = torch_cuda
    sizes = dict(m=40, k=24, n=48)
    rng = np.random.default_rng(2)
    a = rng.uniform(-1, 1, 40 * 24).astype(np.float32)
    b = rng.uniform(-1, 1, 24 * 48).astype(np.float32)
    x = rng.uniform(-1, 1, 48).astype(np.float32)
    bc = host.Binary("mk,kn->mn", sizes, ktype_first_touch=eir.COPY, ktype_last_touch=eir.RELU,
                     aux_outer_sizes=dict(m=1, k=24, n=48))
    out = np.zeros(40 * 48, dtype=np.float32)
    bc.contract(_hp(a), _hp(b), _hp(out), aux=_hp(x))
    ref = np.maximum(a.astype(np.float64).reshape(40, 24) @ b.astype(np.float64).reshape(24, 48) + x, 0.0)
    assert rel_frobenius(ref, out) <= TOL_FP32
    bc.close()
    # ADD first touch: out = out + aux + L*R, the host output's old values are read
    add = host.Binary("mk,kn->mn", sizes, ktype_first_touch=eir.ADD)
    old = rng.uniform(-1, 1, 40 * 48).astype(np.float32)
    aux = rng.uniform(-1, 1, 40 * 48).astype(np.float32)
    out = old.copy()
    add.contract(_hp(a), _hp(b), _hp(out), aux=_hp(aux))
    ref = old.astype(np.float64) + aux + (a.astype(np.float64).reshape(40, 24)
                                          @ b.astype(np.float64).reshape(24, 48)).ravel()
    assert rel_frobenius(ref, out) <= TOL_FP32
    add.close()


@pytest.mark.parametrize("ktype", ["copy", "add"])
def test_unary_host_tensors(torch_cuda, ktype):
    torch = torch_cuda
    u = host.Unary("abcd->dbca", dict(a=8, b=16, c=12, d=20),
                   ktype=eir.COPY if ktype == "copy" else eir.ADD)
    rng = np.random.default_rng(3)
    x = rng.uniform(-1, 1, 8 * 16 * 12 * 20).astype(np.float32)
    y0 = rng.uniform(-1, 1, x.size).astype(np.float32) if ktype == "add" else np.zeros(x.size, np.float32)
    y = y0.copy()
    u.eval(_hp(x), _hp(y))
    ref = x.reshape(8, 16, 12, 20).transpose(3, 1, 2, 0).ravel()
    if ktype == "add":
        ref = y0 + ref
    assert np.array_equal(y, ref)
    u.close()


def test_expression_host_tensors(torch_cuda):
    torch = torch_cuda
    expr = "iae,bf,dcba,cg,dh->hgfei"
    sizes = dict(a=2, b=3, c=4, d=5, e=6, f=7, g=8, h=9, i=10)
    path = [(1, 2), (0, 2), (0, 2), (0, 1)]
    rng = np.random.default_rng(4)
    ins = expr.split("->")[0].split(",")
    numel = lambda t: int(np.prod([sizes[c] for c in t]))
    arrays = [rng.uniform(-1, 1, numel(t)).astype(np.float32) for t in ins]
    # device reference
    dev = [torch.from_numpy(a).cuda() for a in arrays]
    dout = torch.zeros(numel("hgfei"), device="cuda")
    e = host.Expression(expr, sizes, path, dev + [dout])
    e.eval()
    ref = dout.cpu().numpy()
    e.close()
    # all tensors in host memory; one input locked from host memory
    hout = np.zeros(numel("hgfei"), dtype=np.float32)
    e = host.Expression(expr, sizes, path, [_hp(a) for a in arrays] + [_hp(hout)])
    e.store_and_lock_data(2)
    e.eval()
    assert np.array_equal(hout, ref)
    # a second evaluation after the host inputs changed (the locked one keeps its copy)
    arrays[0] *= 2.0
    arrays[2] *= 3.0
    e.eval()
    dev[0] *= 2.0
    e2 = host.Expression(expr, sizes, path, dev + [dout])
    e2.eval()
    assert np.array_equal(hout, dout.cpu().numpy())
    e2.close()
    e.close()


def test_graph_refuses_host_tensors(torch_cuda):
    torch = torch_cuda
    expr, sizes, path = "ab,bc->ac", dict(a=16, b=24, c=32), [(0, 1)]
    a = np.ones(16 * 24, np.float32)
    b = np.ones(24 * 32, np.float32)
    out = np.zeros(16 * 32, np.float32)
    s = torch.cuda.Stream()
    e = host.Expression(expr, sizes, path, [_hp(a), _hp(b), _hp(out)], stream=s)
    with pytest.raises(eir.EinsumIrError) as err:
        e.eval_graph()
    assert err.value.code == eir.NO_DATA_PTR_PROVIDED
    e.eval()
    assert np.array_equal(out, np.full(16 * 32, 24.0, np.float32))
    e.close()
