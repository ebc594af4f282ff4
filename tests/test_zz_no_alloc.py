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
