"""einsum_ir_amd -- MI355X (gfx950) execution backend for einsum_ir's
binary-contraction, permutation and einsum-tree hot path.

The product is native: ``libeinsum_ir_hip.so`` (HIP kernels behind the C ABI
of ``include/einsum_ir_hip.h``) and ``libeinsum_ir.so`` (C++ operator classes
mirroring the reference API: BinaryContraction, Unary, EinsumNode,
EinsumExpression, EinsumTree).  This Python package is a thin ctypes layer
over both for tests and benchmarks; it never computes anything itself.
"""
import ctypes

from . import _lib
from ._lib import (SUCCESS, COMPILATION_FAILED, NO_DATA_PTR_PROVIDED, CALLED_BEFORE_COMPILATION,
                   INVALID_ID, INVALID_BACKEND, INVALID_CPX_DIM, INVALID_DTYPE, INVALID_KTYPE, UNDEFINED_ERROR,
                   FP32, FP64, BF16, UNDEFINED_DTYPE,
                   ZERO, RELU, ADD, COPY, MADD, UNDEFINED_KTYPE, CPX_ZERO, CPX_MADD,
                   DIM_C, DIM_M, DIM_N, DIM_K, DIM_CPX, DIM_I, DIM_J,
                   DTYPE_BYTES, EinsumIrError, hip_lib, check)
from .loops import binary_loops, unary_dims, dim_types, row_major_strides  # noqa: F401


def _ptr(x):
    """Device pointer of a torch tensor, an int, or None."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


def _stream_ptr(stream):
    if stream is None:
        return None
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


class _Plan:
    def __init__(self):
        self._handle = ctypes.c_void_p()

    @property
    def handle(self):
        return self._handle

    def describe(self):
        buf = ctypes.create_string_buffer(512)
        check(hip_lib().etir_hip_plan_describe(self._handle, buf, 512))
        return buf.value.decode()

    @property
    def flops(self):
        return int(hip_lib().etir_hip_plan_flops(self._handle))

    @property
    def bytes(self):
        return int(hip_lib().etir_hip_plan_bytes(self._handle))

    def close(self):
        if self._handle:
            check(hip_lib().etir_hip_plan_destroy(self._handle))
            self._handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class ContractionPlan(_Plan):
    """One binary contraction compiled for the GPU (etir_hip_contraction_create)."""

    def __init__(self, dim_types, sizes, strides_left, strides_right, strides_out,
                 strides_out_aux=None, dtype_left=FP32, dtype_right=FP32, dtype_comp=FP32,
                 dtype_out=FP32, ktype_first_touch=ZERO, ktype_main=MADD,
                 ktype_last_touch=UNDEFINED_KTYPE):
        super().__init__()
        n = len(sizes)
        aux = _lib.i64_array(strides_out_aux) if strides_out_aux is not None else None
        check(hip_lib().etir_hip_contraction_create(
            n, _lib.i32_array(dim_types), _lib.i64_array(sizes), _lib.i64_array(strides_left),
            _lib.i64_array(strides_right), aux, _lib.i64_array(strides_out),
            dtype_left, dtype_right, dtype_comp, dtype_out,
            ktype_first_touch, ktype_main, ktype_last_touch, ctypes.byref(self._handle)))

    def execute(self, left, right, out, aux=None, stream=None):
        check(hip_lib().etir_hip_contraction_execute(self._handle, _ptr(left), _ptr(right),
                                                     _ptr(aux), _ptr(out), _stream_ptr(stream)))


class PermutePlan(_Plan):
    """One permutation compiled for the GPU (etir_hip_permute_create).

    Dims in output order; strides_in already reordered to output order."""

    def __init__(self, sizes, strides_in, strides_out, dtype=FP32, ktype=COPY):
        super().__init__()
        check(hip_lib().etir_hip_permute_create(
            len(sizes), _lib.i64_array(sizes), _lib.i64_array(strides_in),
            _lib.i64_array(strides_out), dtype, dtype, dtype, ktype, ctypes.byref(self._handle)))

    def execute(self, inp, out, stream=None):
        check(hip_lib().etir_hip_permute_execute(self._handle, _ptr(inp), _ptr(out),
                                                 _stream_ptr(stream)))


def synchronize(stream=None):
    check(hip_lib().etir_hip_synchronize(_stream_ptr(stream)))


def device_count():
    return int(hip_lib().etir_hip_device_count())
