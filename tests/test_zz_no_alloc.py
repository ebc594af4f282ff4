"""GPU checks of the allocation-free entry point
etir_hip_contraction_execute_noalloc (include/einsum_ir_hip.h), called
through the C ABI.  Its results must equal those of the allocating path
(etir_hip_contraction_create + etir_hip_contraction_execute) bit for bit:
both run the same kernels over the same offset tables in the same order, the
tables here generated on the device, there copied from the host.  Two calls
in a row share the scratch array, the second with a smaller input, so stale
tables or partial sums from the first call would show."""
import ctypes

import numpy as np
import pytest

import einsum_ir_amd as eir
from einsum_ir_amd import _lib
from tests.helpers import loops_for, parse_binary, tensor_numel, rel_frobenius, TOL_FP32, TOL_BF16

pytestmark = pytest.mark.gpu

_i64p = ctypes.POINTER(ctypes.c_int64)
_i32p = ctypes.POINTER(ctypes.c_int32)


def _last_error():
    msg = eir.hip_lib().etir_hip_last_error()
    return msg.decode() if msg else ""


def _noalloc_fn():
    lib = eir.hip_lib()
    fn = lib.etir_hip_contraction_execute_noalloc
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int64, _i32p, _i64p, _i64p, _i64p, _i64p, _i64p] + [ctypes.c_int32] * 7 \
        + [ctypes.c_void_p] * 5
    return fn


def _inputs(torch, expr, sizes, dtype, seed):
    left, right, out = parse_binary(expr)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    tdt = torch.bfloat16 if dtype == eir.BF16 else torch.float32
    a = (torch.rand(tensor_numel(left, sizes), device="cuda", generator=g) * 2 - 1).to(tdt)
    b = (torch.rand(tensor_numel(right, sizes), device="cuda", generator=g) * 2 - 1).to(tdt)
    return a, b, tensor_numel(out, sizes)


def _run_both(torch, expr, sizes, dtype=eir.FP32, seed=0):
    loops = loops_for(expr, sizes)
    a, b, n_out = _inputs(torch, expr, sizes, dtype, seed)
    stream = torch.cuda.current_stream()
    # allocating path
    plan = eir.ContractionPlan(loops["dim_types"], loops["sizes"], loops["strides_left"],
                               loops["strides_right"], loops["strides_out"],
                               dtype_left=dtype, dtype_right=dtype)
    desc = plan.describe()
    ref = torch.full((n_out,), float("nan"), device="cuda")
    plan.execute(a, b, ref, stream=stream)
    plan.close()
    # allocation-free path, output pre-filled with NaN
    got = torch.full((n_out,), float("nan"), device="cuda")
    n = len(loops["sizes"])
    rc = _noalloc_fn()(n, _lib.i32_array(loops["dim_types"]), _lib.i64_array(loops["sizes"]),
                       _lib.i64_array(loops["strides_left"]), _lib.i64_array(loops["strides_right"]),
                       None, _lib.i64_array(loops["strides_out"]),
                       dtype, dtype, eir.FP32, eir.FP32, eir.ZERO, eir.MADD, eir.UNDEFINED_KTYPE,
                       a.data_ptr(), b.data_ptr(), None, got.data_ptr(), stream.cuda_stream)
    assert rc == 0, _last_error()
    torch.cuda.synchronize()
    return ref.cpu().numpy(), got.cpu().numpy(), desc, (a, b)


def test_noalloc_two_calls_match_allocating_path(torch_cuda):
    torch = torch_cuda
    # 1: few output tiles and a long K (split-K: 8 MB of partial sums in the scratch array)
    ref1, got1, desc1, _ = _run_both(torch, "mk,kn->mn", dict(m=64, k=8192, n=512), seed=1)
    assert "split-K" in desc1, desc1
    assert np.array_equal(ref1, got1), "first call differs from the allocating path"
    # 2: a smaller split-K contraction over the same scratch (other tables, fewer slices)
    ref2, got2, desc2, (a2, b2) = _run_both(torch, "mk,kn->mn", dict(m=96, k=4096, n=160), seed=2)
    assert "split-K" in desc2, desc2
    assert np.array_equal(ref2, got2), "second call differs from the allocating path"
    exact = a2.double().cpu().numpy().reshape(96, 4096) @ b2.double().cpu().numpy().reshape(4096, 160)
    assert rel_frobenius(exact, got2) <= TOL_FP32


def test_noalloc_bf16_layout(torch_cuda):
    """A bf16 contraction with the config-3 layout (no workspace: tables only),
    then again after a larger call left other tables in the array."""
    torch = torch_cuda
    sizes = dict(z=2, a=4, m=64, b=4, n=64, k=256)
    ref, got, _, (a, b) = _run_both(torch, "zakm,zbkn->zabmn", sizes, dtype=eir.BF16, seed=3)
    assert np.array_equal(ref, got)
    A = a.float().cpu().numpy().astype(np.float64).reshape(2, 4, 256, 64)
    B = b.float().cpu().numpy().astype(np.float64).reshape(2, 4, 256, 64)
    exact = np.einsum("zakm,zbkn->zabmn", A, B).ravel()
    assert rel_frobenius(exact, got) <= TOL_BF16


def _run_both_aux(torch, expr, sizes, aux_outer, first, last, seed):
    """As _run_both, with an aux tensor (first touch COPY/ADD or last touch
    ADD) whose outer sizes broadcast it; returns both outputs, the plan's
    description and the inputs."""
    loops = loops_for(expr, sizes, sizes_outer_aux=aux_outer)
    a, b, n_out = _inputs(torch, expr, sizes, eir.FP32, seed)
    _, _, out = parse_binary(expr)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 100)
    x = torch.rand(tensor_numel(out, aux_outer), device="cuda", generator=g) * 2 - 1
    # first touch ADD adds to what the output holds: both start from the same
    # values (NaN otherwise, so that an unwritten element shows)
    init = (torch.rand(n_out, device="cuda", generator=g) * 2 - 1) if first == eir.ADD \
        else torch.full((n_out,), float("nan"), device="cuda")
    stream = torch.cuda.current_stream()
    plan = eir.ContractionPlan(loops["dim_types"], loops["sizes"], loops["strides_left"],
                               loops["strides_right"], loops["strides_out"],
                               strides_out_aux=loops["strides_out_aux"], ktype_first_touch=first,
                               ktype_last_touch=last)
    desc = plan.describe()
    ref = init.clone()
    plan.execute(a, b, ref, aux=x, stream=stream)
    plan.close()
    got = init.clone()
    rc = _noalloc_fn()(len(loops["sizes"]), _lib.i32_array(loops["dim_types"]), _lib.i64_array(loops["sizes"]),
                       _lib.i64_array(loops["strides_left"]), _lib.i64_array(loops["strides_right"]),
                       _lib.i64_array(loops["strides_out_aux"]), _lib.i64_array(loops["strides_out"]),
                       eir.FP32, eir.FP32, eir.FP32, eir.FP32, first, eir.MADD, last,
                       a.data_ptr(), b.data_ptr(), x.data_ptr(), got.data_ptr(), stream.cuda_stream)
    assert rc == 0, _last_error()
    torch.cuda.synchronize()
    return ref.cpu().numpy(), got.cpu().numpy(), desc, (a, b, x)


def test_noalloc_aux_and_k_tables(torch_cuda):
    """The device-side fills of the aux tables and of a K that is not one
    affine index (K = (k, l) with l outermost in the right operand): a bias
    broadcast over the rows (first touch COPY, last touch RELU), then a
    column-broadcast aux with first touch ADD over the same scratch array.
    Bit for bit against create + execute, and the first against float64."""
    torch = torch_cuda
    sizes1 = dict(m=96, k=12, l=20, n=200)
    ref1, got1, desc1, (a1, b1, x1) = _run_both_aux(torch, "mkl,lkn->mn", sizes1, dict(m=1, n=200),
                                                     eir.COPY, eir.RELU, seed=5)
    assert "k_affine=0" in desc1, desc1
    assert np.array_equal(ref1, got1), "aux/K-table call differs from the allocating path"
    A = a1.double().cpu().numpy().reshape(96, 12, 20)
    B = b1.double().cpu().numpy().reshape(20, 12, 200)
    exact = np.maximum(np.einsum("mkl,lkn->mn", A, B) + x1.double().cpu().numpy().reshape(1, 200), 0.0)
    assert rel_frobenius(exact.ravel(), got1) <= TOL_FP32
    sizes2 = dict(m=40, k=6, l=16, n=72)
    ref2, got2, desc2, _ = _run_both_aux(torch, "mkl,lkn->mn", sizes2, dict(m=40, n=1), eir.ADD,
                                         eir.UNDEFINED_KTYPE, seed=6)
    assert "k_affine=0" in desc2, desc2
    assert not np.isnan(got2).any()
    assert np.array_equal(ref2, got2), "second aux/K-table call differs from the allocating path"


def test_noalloc_rejects_oversized_plan(torch_cuda):
    """Offset tables beyond the 64 MiB array: a clear error, nothing launched."""
    torch = torch_cuda
    m = 6_000_000          # M tables: 3 x 4 bytes x 6M entries = 72 MB
    loops = loops_for("mk,kn->mn", dict(m=m, k=2, n=2))
    a = torch.zeros(2 * m, device="cuda")
    b = torch.zeros(4, device="cuda")
    out = torch.zeros(2 * m, device="cuda")
    rc = _noalloc_fn()(len(loops["sizes"]), _lib.i32_array(loops["dim_types"]), _lib.i64_array(loops["sizes"]),
                       _lib.i64_array(loops["strides_left"]), _lib.i64_array(loops["strides_right"]),
                       None, _lib.i64_array(loops["strides_out"]),
                       eir.FP32, eir.FP32, eir.FP32, eir.FP32, eir.ZERO, eir.MADD, eir.UNDEFINED_KTYPE,
                       a.data_ptr(), b.data_ptr(), None, out.data_ptr(),
                       torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc != 0
    msg = _last_error()
    assert "scratch" in msg and str(64 << 20) in msg, msg
