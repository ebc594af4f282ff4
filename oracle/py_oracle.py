"""TEST INFRASTRUCTURE ONLY -- numpy binding of oracle/liboracle.so.

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
and never by the product package.  See oracle.c for what each function
restates and how it is pinned.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

FP32, FP64, BF16 = 0, 1, 2
ZERO, RELU, ADD, COPY, MADD, UNDEF = 0, 1, 2, 3, 4, 99

_i64p = ctypes.POINTER(ctypes.c_int64)
_i32p = ctypes.POINTER(ctypes.c_int32)
_vp = ctypes.c_void_p
_lib = None


def build():
    """Compiles liboracle.so (gcc) from oracle.c."""
    subprocess.check_call(["make", "-s", "-C", _HERE])


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        l = ctypes.CDLL(LIB_PATH)
        l.oracle_contract.restype = ctypes.c_int
        l.oracle_contract.argtypes = [ctypes.c_int64, _i32p, _i64p, _i64p, _i64p, _i64p, _i64p,
                                      ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                      ctypes.c_int32, ctypes.c_int32, _vp, _vp, _vp, _vp]
        l.oracle_contract_blocked.restype = ctypes.c_int
        l.oracle_contract_blocked.argtypes = [ctypes.c_int64, _i32p, _i64p, _i64p, _i64p, _i64p, _i64p,
                                              ctypes.c_int32, ctypes.c_int32, _vp, _vp, _vp, _vp,
                                              ctypes.c_int32]
        l.oracle_permute_blocked.restype = ctypes.c_int
        l.oracle_permute_blocked.argtypes = [ctypes.c_int64, _i64p, _i64p, _i64p, _vp, _vp]
        l.oracle_permute.restype = ctypes.c_int
        l.oracle_permute.argtypes = [ctypes.c_int64, _i64p, _i64p, _i64p, ctypes.c_int32,
                                     ctypes.c_int32, _vp, _vp, ctypes.c_int32]
        l.oracle_f32_to_bf16.restype = None
        l.oracle_f32_to_bf16.argtypes = [_vp, _vp, ctypes.c_int64]
        l.oracle_bf16_to_f32.restype = None
        l.oracle_bf16_to_f32.argtypes = [_vp, _vp, ctypes.c_int64]
        _lib = l
    return _lib


def _a64(v):
    v = list(v)
    return (ctypes.c_int64 * max(1, len(v)))(*v)


def _a32(v):
    v = list(v)
    return (ctypes.c_int32 * max(1, len(v)))(*v)


def _np_ptr(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"] or a.ndim <= 1
    return a.ctypes.data


def contract(loops, left, right, out, aux=None, dtype_left=FP32, dtype_right=FP32,
             dtype_out=FP32, first_touch=ZERO, last_touch=UNDEF):
    """Exact (fp64-accumulating) contraction over the loop IR; writes `out` in place.

    loops: dict with dim_types, sizes, strides_left/right/out(/out_aux) in elements.
    Arrays are flat numpy buffers (uint16 for bf16)."""
    aux_s = loops.get("strides_out_aux")
    rc = lib().oracle_contract(len(loops["sizes"]), _a32(loops["dim_types"]), _a64(loops["sizes"]),
                               _a64(loops["strides_left"]), _a64(loops["strides_right"]),
                               _a64(aux_s) if aux_s is not None else None,
                               _a64(loops["strides_out"]),
                               dtype_left, dtype_right, dtype_out, first_touch, last_touch,
                               _np_ptr(left), _np_ptr(right), _np_ptr(aux), _np_ptr(out))
    assert rc == 0
    return out


def contract_blocked(loops, left, right, out, aux=None, first_touch=ZERO, last_touch=UNDEF,
                     num_threads=0):
    """OpenMP blocked fp32 restatement of the reference CPU algorithm (baseline)."""
    aux_s = loops.get("strides_out_aux")
    for a in (left, right, out):
        assert a.dtype == np.float32
    rc = lib().oracle_contract_blocked(len(loops["sizes"]), _a32(loops["dim_types"]), _a64(loops["sizes"]),
                                       _a64(loops["strides_left"]), _a64(loops["strides_right"]),
                                       _a64(aux_s) if aux_s is not None else None,
                                       _a64(loops["strides_out"]), first_touch, last_touch,
                                       _np_ptr(left), _np_ptr(right), _np_ptr(aux), _np_ptr(out),
                                       num_threads)
    assert rc == 0
    return out


def permute(sizes, strides_in, strides_out, inp, out, dtype=FP32, ktype=COPY, num_threads=0):
    """Permutation with COPY / ZERO / ADD; dims in output order."""
    rc = lib().oracle_permute(len(sizes), _a64(sizes), _a64(strides_in), _a64(strides_out),
                              dtype, ktype, _np_ptr(inp), _np_ptr(out), num_threads)
    assert rc == 0
    return out


def permute_blocked(sizes, strides_in, strides_out, inp, out):
    """fp32 COPY permutation by the blocked CPU baseline (dims in output
    order); returns False for layouts it does not cover."""
    rc = lib().oracle_permute_blocked(len(sizes), _a64(sizes), _a64(strides_in), _a64(strides_out),
                                      _np_ptr(inp), _np_ptr(out))
    assert rc in (0, 2)
    return rc == 0


def f32_to_bf16(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_bf16(x.ctypes.data, out.ctypes.data, x.size)
    return out


def bf16_to_f32(b):
    b = np.ascontiguousarray(b, dtype=np.uint16)
    out = np.empty(b.shape, dtype=np.float32)
    lib().oracle_bf16_to_f32(b.ctypes.data, out.ctypes.data, b.size)
    return out


def _names_sorted(names):
    def key(n):
        try:
            return (0, int(n), "")
        except ValueError:
            return (1, 0, n)
    return sorted(names, key=key)


def contract_path(expr, sizes, path, arrays, dtype=FP64, round_bf16=False):
    """Einsum expression evaluated pairwise along a contraction path
    (opt_einsum standard form) with oracle_contract for every step; each
    intermediate keeps the dims still needed later in ascending name order,
    as EinsumExpression::substring_out does (reference
    src/frontend/EinsumExpression.cpp:25-70).  Returns the output as float64.
    round_bf16: every step's result is rounded to bfloat16 (RNE), as a tree
    whose tensors are bf16 stores its intermediates and output.
    Pinned by tests/test_oracle.py: numpy.einsum in float64, and for
    round_bf16 numpy.einsum steps with torch's bfloat16 conversion between.

    arrays: flat numpy arrays of the inputs in their expression layouts."""
    lhs, out = expr.replace(" ", "").split("->")
    live = [(list(t), np.ascontiguousarray(a, dtype=np.float64)) for t, a in zip(lhs.split(","), arrays)]

    def strides_of(dims):
        st, acc = {}, 1
        for d in reversed(dims):
            st[d] = acc if sizes[d] >= 2 else 0
            acc *= sizes[d]
        return st

    for step, (i, j) in enumerate(path):
        (dl, al), (dr, ar) = live[i], live[j]
        rest = [d for k, (t, _) in enumerate(live) if k not in (i, j) for d in t] + list(out)
        last = step == len(path) - 1
        res = list(out) if last else _names_sorted(set(d for d in dl + dr if d in rest))
        sl, sr, so = strides_of(dl), strides_of(dr), strides_of(res)
        alld = list(dict.fromkeys(res + dl + dr))
        types = []
        for d in alld:
            in_l, in_r, in_o = d in dl, d in dr, d in res
            types.append(0 if (in_l and in_r and in_o) else 1 if (in_l and in_o) else
                         2 if (in_r and in_o) else 3 if (in_l and in_r) else 5 if in_l else 6)
        loops = dict(dim_types=types, sizes=[sizes[d] for d in alld],
                     strides_left=[sl.get(d, 0) for d in alld], strides_right=[sr.get(d, 0) for d in alld],
                     strides_out=[so.get(d, 0) for d in alld])
        o = np.zeros(int(np.prod([sizes[d] for d in res])) if res else 1, dtype=np.float64)
        contract(loops, al, ar, o, dtype_left=FP64, dtype_right=FP64, dtype_out=FP64)
        if round_bf16:
            o = bf16_to_f32(f32_to_bf16(o.astype(np.float32))).astype(np.float64)
        live = [t for k, t in enumerate(live) if k not in (i, j)] + [(res, o)]
    return live[0][1]
