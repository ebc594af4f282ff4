"""ctypes binding of ``libeinsum_ir_hip.so`` (C ABI in include/einsum_ir_hip.h).

This is plumbing for Python callers (tests, bench.py): it loads the in-tree
native library and fails loudly when it is missing -- there is no Python or
CPU fallback for any operation.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_HIP_PATH = os.path.join(_HERE, "libeinsum_ir_hip.so")
LIB_HOST_PATH = os.path.join(_HERE, "libeinsum_ir.so")

# error codes, dtypes, kernel and dimension types (einsum_ir enums, src/constants.h)
SUCCESS = 0
COMPILATION_FAILED = 1
NO_DATA_PTR_PROVIDED = 4
CALLED_BEFORE_COMPILATION = 5
INVALID_ID = 6
INVALID_BACKEND = 7
INVALID_CPX_DIM = 8
INVALID_DTYPE = 9
INVALID_KTYPE = 10
UNDEFINED_ERROR = 99

FP32, FP64, BF16, UNDEFINED_DTYPE = 0, 1, 2, 99
ZERO, RELU, ADD, COPY, MADD, UNDEFINED_KTYPE = 0, 1, 2, 3, 4, 99
CPX_ZERO, CPX_MADD = 6, 8
DIM_C, DIM_M, DIM_N, DIM_K, DIM_CPX, DIM_I, DIM_J = 0, 1, 2, 3, 4, 5, 6

DTYPE_BYTES = {FP32: 4, FP64: 8, BF16: 2}

_i64p = ctypes.POINTER(ctypes.c_int64)
_i32p = ctypes.POINTER(ctypes.c_int32)
_vp = ctypes.c_void_p

_HIP_SIGS = {
    "etir_hip_contraction_create": (ctypes.c_int, [ctypes.c_int64, _i32p, _i64p, _i64p, _i64p, _i64p, _i64p,
                                                   ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                                   ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                                   ctypes.POINTER(_vp)]),
    "etir_hip_contraction_execute": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp]),
    "etir_hip_permute_create": (ctypes.c_int, [ctypes.c_int64, _i64p, _i64p, _i64p, ctypes.c_int32,
                                               ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                               ctypes.POINTER(_vp)]),
    "etir_hip_permute_execute": (ctypes.c_int, [_vp, _vp, _vp, _vp]),
    "etir_hip_plan_destroy": (ctypes.c_int, [_vp]),
    "etir_hip_plan_describe": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.c_int64]),
    "etir_hip_plan_flops": (ctypes.c_int64, [_vp]),
    "etir_hip_plan_bytes": (ctypes.c_int64, [_vp]),
    "etir_hip_last_error": (ctypes.c_char_p, []),
    "etir_hip_malloc": (ctypes.c_int, [ctypes.POINTER(_vp), ctypes.c_int64]),
    "etir_hip_free": (ctypes.c_int, [_vp]),
    "etir_hip_memcpy_h2d": (ctypes.c_int, [_vp, _vp, ctypes.c_int64]),
    "etir_hip_memcpy_d2h": (ctypes.c_int, [_vp, _vp, ctypes.c_int64]),
    "etir_hip_memcpy_d2d": (ctypes.c_int, [_vp, _vp, ctypes.c_int64, _vp]),
    "etir_hip_memset": (ctypes.c_int, [_vp, ctypes.c_int32, ctypes.c_int64]),
    "etir_hip_synchronize": (ctypes.c_int, [_vp]),
    "etir_hip_device_count": (ctypes.c_int, []),
    "etir_hip_pointer_is_device": (ctypes.c_int, [_vp]),
    "etir_hip_stream_create": (ctypes.c_int, [ctypes.POINTER(ctypes.c_void_p)]),
    "etir_hip_stream_destroy": (ctypes.c_int, [ctypes.c_void_p]),
    "etir_hip_graph_begin": (ctypes.c_int, [ctypes.c_void_p]),
    "etir_hip_graph_end": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]),
    "etir_hip_graph_abort": (ctypes.c_int, [ctypes.c_void_p]),
    "etir_hip_graph_launch": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
    "etir_hip_graph_destroy": (ctypes.c_int, [ctypes.c_void_p]),
    "etir_hip_event_create": (ctypes.c_int, [ctypes.POINTER(ctypes.c_void_p)]),
    "etir_hip_event_destroy": (ctypes.c_int, [ctypes.c_void_p]),
    "etir_hip_event_record": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
    "etir_hip_stream_wait_event": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
}

_lib_hip = None


class EinsumIrError(RuntimeError):
    """Raised when a native call returns an einsum_ir error code."""

    def __init__(self, code, msg):
        super().__init__(f"einsum_ir error {code}: {msg}")
        self.code = code


def hip_lib():
    """Loads libeinsum_ir_hip.so (in-tree); raises if it has not been built."""
    global _lib_hip
    if _lib_hip is None:
        if not os.path.exists(LIB_HIP_PATH):
            raise ImportError(f"{LIB_HIP_PATH} is missing: run __graft_entry__.build() "
                              "(make -C einsum_ir_amd) first; there is no fallback path")
        lib = ctypes.CDLL(LIB_HIP_PATH)
        for name, (res, args) in _HIP_SIGS.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib_hip = lib
    return _lib_hip


def check(code):
    if code != SUCCESS:
        msg = hip_lib().etir_hip_last_error()
        raise EinsumIrError(code, msg.decode() if msg else "")


def i64_array(values):
    values = list(values)
    return (ctypes.c_int64 * max(1, len(values)))(*values)


def i32_array(values):
    values = list(values)
    return (ctypes.c_int32 * max(1, len(values)))(*values)
