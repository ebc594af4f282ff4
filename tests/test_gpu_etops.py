"""GPU parity of the etops-compatible API (einsum_ir_amd.etops) on the HIP
backend: TensorOperation built from a TensorOperationConfig, executed on
device arrays (torch tensors, DLPack objects, raw pointers) and on host numpy
arrays (staged), as the reference's etops module is used (reference
python/src/etops/__init__.py, python/src/TensorOperation.cpp:220-479).

Checker: the CPU oracle on the same loop IR (oracle_contract accumulates in
fp64; oracle_permute is exact).  Bars: fp32 relative Frobenius <= 1e-5, bf16
<= 2e-3, permutations bit-exact.
"""
import numpy as np
import pytest

from einsum_ir_amd import etops
from tests.helpers import TOL_BF16, TOL_FP32, rel_frobenius

pytestmark = pytest.mark.gpu

C, M, N, K = etops.dim.c, etops.dim.m, etops.dim.n, etops.dim.k


def _config(dim_types, sizes, s0, s1, s2, first=etops.prim.zero, last=etops.prim.none,
            main=etops.prim.gemm, dtype=etops.float32):
    return etops.TensorOperationConfig(data_type=dtype, prim_first=first, prim_main=main, prim_last=last,
                                       dim_types=tuple(dim_types), exec_types=(etops.exec.seq,) * len(sizes),
                                       dim_sizes=tuple(sizes), strides=((tuple(s0), tuple(s1), tuple(s2)),))


def _extent(sizes, strides):
    return 1 + sum((s - 1) * st for s, st in zip(sizes, strides))


def _oracle(oracle, cfg, a, b, out, first, last):
    loops = dict(dim_types=[int(d) for d in cfg.dim_types], sizes=list(cfg.dim_sizes),
                 strides_left=list(cfg.strides[0][0]), strides_right=list(cfg.strides[0][1]),
                 strides_out=list(cfg.strides[0][2]))
    return oracle.contract(loops, a, b, out, first_touch=first, last_touch=last)


def test_gemm_column_major_torch_device(torch_cuda, oracle):
    """C[m,n] += ... column-major GEMM (m fastest), loops (m, n, k)."""
    torch = torch_cuda
    m, n, k = 96, 80, 72
    cfg = _config((M, N, K), (m, n, k), (1, 0, m), (0, k, 1), (1, m, 0))
    rng = np.random.default_rng(1)
    a = rng.uniform(-1, 1, m * k).astype(np.float32)
    b = rng.uniform(-1, 1, k * n).astype(np.float32)
    op = etops.TensorOperation(cfg)
    assert "contract" in op.describe()
    da, db = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    dout = torch.full((m * n,), float("nan"), device="cuda")
    op.execute(da, db, dout)
    ref = _oracle(oracle, cfg, a, b, np.zeros(m * n, np.float32), oracle.ZERO, oracle.UNDEF)
    assert rel_frobenius(ref, dout.cpu().numpy()) <= TOL_FP32
    op.close()


def test_batched_brgemm_relu_numpy_staged(oracle):
    """c dim + brgemm + ReLU last touch, host numpy arrays (staged)."""
    c, m, n, br, k = 3, 40, 24, 4, 16
    # in0[c][br][k][m], in1[c][br][n][k], out[c][n][m]
    s_in0 = (br * k * m, 1, 0, k * m, m)
    s_in1 = (br * n * k, 0, k, n * k, 1)
    s_out = (n * m, 1, m, 0, 0)
    cfg = _config((C, M, N, K, K), (c, m, n, br, k), s_in0, s_in1, s_out,
                  main=etops.prim.brgemm, last=etops.prim.relu)
    rng = np.random.default_rng(2)
    a = rng.uniform(-1, 1, c * br * k * m).astype(np.float32)
    b = rng.uniform(-1, 1, c * br * n * k).astype(np.float32)
    out = np.full(c * n * m, np.nan, np.float32)
    etops.TensorOperation(cfg).execute(a, b, out)
    ref = _oracle(oracle, cfg, a, b, np.zeros_like(out), oracle.ZERO, oracle.RELU)
    assert rel_frobenius(ref, out) <= TOL_FP32
    assert (out >= 0).all() and (out == 0).any()


def test_prim_first_none_accumulates(torch_cuda, oracle):
    """prim_first none: the product is added to the output's old values."""
    torch = torch_cuda
    m, n, k = 64, 64, 40
    cfg = _config((N, M, K), (n, m, k), (0, k, 1), (k, 0, 1), (m, 1, 0), first=etops.prim.none)
    rng = np.random.default_rng(3)
    a = rng.uniform(-1, 1, m * k).astype(np.float32)
    b = rng.uniform(-1, 1, n * k).astype(np.float32)
    init = rng.uniform(-1, 1, n * m).astype(np.float32)
    dout = torch.from_numpy(init.copy()).cuda()
    etops.TensorOperation(cfg).execute(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda(), dout)
    ref = _oracle(oracle, cfg, a, b, init.copy(), oracle.UNDEF, oracle.UNDEF)
    assert rel_frobenius(ref, dout.cpu().numpy()) <= TOL_FP32


def test_bfloat16_device_arrays(torch_cuda, oracle):
    torch = torch_cuda
    m, n, k = 128, 136, 64
    cfg = _config((M, N, K), (m, n, k), (1, 0, m), (0, k, 1), (1, m, 0), dtype=etops.bfloat16)
    rng = np.random.default_rng(4)
    a = rng.uniform(-1, 1, m * k).astype(np.float32)
    b = rng.uniform(-1, 1, k * n).astype(np.float32)
    da = torch.from_numpy(a).cuda().to(torch.bfloat16)
    db = torch.from_numpy(b).cuda().to(torch.bfloat16)
    dout = torch.zeros(m * n, dtype=torch.bfloat16, device="cuda")
    etops.TensorOperation(cfg).execute(da, db, dout)
    a16 = da.view(torch.int16).cpu().numpy().view(np.uint16)
    b16 = db.view(torch.int16).cpu().numpy().view(np.uint16)
    loops = dict(dim_types=[1, 2, 3], sizes=[m, n, k], strides_left=[1, 0, m], strides_right=[0, k, 1],
                 strides_out=[1, m, 0])
    ref = oracle.contract(loops, a16, b16, np.zeros(m * n, np.float32), dtype_left=oracle.BF16,
                          dtype_right=oracle.BF16)
    assert rel_frobenius(ref, dout.float().cpu().numpy()) <= TOL_BF16


def test_dlpack_and_raw_pointers(torch_cuda, oracle):
    torch = torch_cuda

    class DlpackOnly:
        def __init__(self, t):
            self._t = t

        def __dlpack__(self, stream=None):
            return self._t.__dlpack__()

        def __dlpack_device__(self):
            return self._t.__dlpack_device__()

    m, n, k = 32, 48, 24
    cfg = _config((M, N, K), (m, n, k), (1, 0, m), (0, k, 1), (1, m, 0))
    rng = np.random.default_rng(5)
    a = rng.uniform(-1, 1, m * k).astype(np.float32)
    b = rng.uniform(-1, 1, k * n).astype(np.float32)
    da, db = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    dout = torch.zeros(m * n, device="cuda")
    op = etops.TensorOperation(cfg)
    op.execute(DlpackOnly(da), db.data_ptr(), DlpackOnly(dout))
    ref = _oracle(oracle, cfg, a, b, np.zeros(m * n, np.float32), oracle.ZERO, oracle.UNDEF)
    assert rel_frobenius(ref, dout.cpu().numpy()) <= TOL_FP32
    dout.zero_()
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    op.execute_async(da, db, dout, stream=s)
    s.synchronize()
    assert rel_frobenius(ref, dout.cpu().numpy()) <= TOL_FP32
    with pytest.raises(TypeError):
        op.execute_async(a, db, dout)      # host arrays need execute()


@pytest.mark.parametrize("dtype,npt", [(etops.float32, np.float32), (etops.float64, np.float64)])
def test_unary_transpose_and_zero(torch_cuda, dtype, npt):
    """copy: bit-exact 3-D permutation; zero: all zeros (numpy host arrays
    and device tensors)."""
    torch = torch_cuda
    d0, d1, d2 = 33, 20, 17
    x = np.random.default_rng(6).uniform(-1, 1, (d0, d1, d2)).astype(npt)
    # out[d2][d0][d1] = in[d0][d1][d2]; dims listed as (d0, d1, d2)
    s_in = (d1 * d2, d2, 1)
    s_out = (d1, 1, d0 * d1)
    cfg = etops.TensorOperationConfig(data_type=dtype, prim_first=etops.prim.none, prim_main=etops.prim.copy,
                                      prim_last=etops.prim.none, dim_types=(C, C, C),
                                      exec_types=(etops.exec.seq,) * 3, dim_sizes=(d0, d1, d2),
                                      strides=((s_in, s_out),))
    out = np.full(d0 * d1 * d2, np.nan, npt)
    op = etops.TensorOperation(cfg)
    op.execute(x.reshape(-1), None, out)
    assert np.array_equal(out.reshape(d2, d0, d1), np.transpose(x, (2, 0, 1)))
    dout = torch.full((d0 * d1 * d2,), 7.0, dtype=torch.float32 if npt == np.float32 else torch.float64,
                      device="cuda")
    op.execute(torch.from_numpy(x.reshape(-1)).cuda(), None, dout)
    assert np.array_equal(dout.cpu().numpy().reshape(d2, d0, d1), np.transpose(x, (2, 0, 1)))
    zcfg = etops.TensorOperationConfig(**{**cfg.__dict__, "prim_main": etops.prim.zero})
    etops.TensorOperation(zcfg).execute(torch.from_numpy(x.reshape(-1)).cuda(), None, dout)
    assert not dout.cpu().numpy().any()


def test_float64_contraction_and_setup_errors(torch_cuda, oracle):
    torch = torch_cuda
    m, n, k = 24, 40, 12
    cfg = _config((M, N, K), (m, n, k), (1, 0, m), (0, k, 1), (1, m, 0), dtype=etops.float64,
                  last=etops.prim.relu)
    rng = np.random.default_rng(8)
    a, b = rng.uniform(-1, 1, m * k), rng.uniform(-1, 1, k * n)
    dout = torch.zeros(m * n, dtype=torch.float64, device="cuda")
    etops.TensorOperation(cfg).execute(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda(), dout)
    loops = dict(dim_types=[1, 2, 3], sizes=[m, n, k], strides_left=[1, 0, m], strides_right=[0, k, 1],
                 strides_out=[1, m, 0])
    ref = oracle.contract(loops, a, b, np.zeros(m * n), dtype_left=oracle.FP64, dtype_right=oracle.FP64,
                          dtype_out=oracle.FP64, last_touch=oracle.RELU)
    assert rel_frobenius(ref, dout.cpu().numpy()) <= 1e-12
    op = etops.TensorOperation()
    assert op.setup("tpp", cfg.data_type, cfg.prim_first, cfg.prim_main, cfg.prim_last, cfg.dim_types,
                    cfg.exec_types, cfg.dim_sizes, cfg.strides) == etops.ErrorType.compilation_failed
    assert op.setup(None, etops.float32, cfg.prim_first, cfg.prim_main, cfg.prim_last, cfg.dim_types,
                    cfg.exec_types, cfg.dim_sizes, (cfg.strides[0][:2],)) == etops.ErrorType.invalid_stride_shape
    assert op.setup("hip", cfg.data_type, cfg.prim_first, etops.prim.relu, cfg.prim_last, cfg.dim_types,
                    cfg.exec_types, cfg.dim_sizes, cfg.strides) == etops.ErrorType.compilation_failed
    with pytest.raises(RuntimeError, match="execute before a successful setup"):
        op.execute(torch.zeros(1, device="cuda"), torch.zeros(1, device="cuda"), dout)


def test_optimized_config_runs_the_same(torch_cuda, oracle):
    """etops.optimize's fused loops (b,c / m1,m2 / k1,k2 contiguous in every
    tensor, a size-1 loop dropped) give the same output bit for bit as the
    config it came from, and both match the oracle."""
    torch = torch_cuda
    sizes = (2, 3, 40, 1, 5, 48, 7, 8)
    types = (C, C, M, N, M, N, K, K)
    sa = (3360 * 10, 1120 * 10, 280, 0, 56, 0, 8, 1)
    sb = (1008 * 8, 336 * 8, 0, 0, 0, 56, 8, 1)
    so = (360 * 80, 120 * 80, 30 * 8, 0, 6 * 8, 1, 0, 0)
    cfg = _config(types, sizes, sa, sb, so)
    opt = etops.optimize(cfg)
    assert opt.dim_types == (C, M, N, K) and opt.dim_sizes == (6, 200, 48, 56), opt
    rng = np.random.default_rng(5)
    a = rng.uniform(-1, 1, _extent(sizes, sa)).astype(np.float32)
    b = rng.uniform(-1, 1, _extent(sizes, sb)).astype(np.float32)
    n_out = _extent(sizes, so)
    da, db = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    outs = []
    for c in (cfg, opt):
        op = etops.TensorOperation(c)
        dout = torch.full((n_out,), float("nan"), device="cuda")
        op.execute(da, db, dout)
        op.close()
        outs.append(dout.cpu().numpy())
    assert np.array_equal(outs[0], outs[1])
    ref = _oracle(oracle, cfg, a, b, np.zeros(n_out, np.float32), oracle.ZERO, oracle.UNDEF)
    assert rel_frobenius(ref, outs[1]) <= TOL_FP32
