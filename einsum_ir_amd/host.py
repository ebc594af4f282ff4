"""ctypes binding of ``libeinsum_ir.so`` (include/einsum_ir.h): the C++
operator classes -- BinaryContractionHip, UnaryHip, EinsumExpression,
EinsumTree -- driven from Python with device tensors (torch) or raw pointers.
"""
import ctypes
import os
import re

from . import _lib

_i64p = ctypes.POINTER(ctypes.c_int64)
_vp = ctypes.c_void_p
_lib_host = None

_SIGS = {
    "etir_binary_create": (ctypes.c_int, [ctypes.c_char_p, _i64p, ctypes.c_int64, _i64p, ctypes.c_int32,
                                          ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                          ctypes.c_int32, ctypes.c_int32, ctypes.POINTER(_vp)]),
    "etir_binary_contract": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp]),
    "etir_binary_num_ops": (ctypes.c_int64, [_vp]),
    "etir_binary_sizes": (ctypes.c_int, [_vp, _i64p, _i64p]),
    "etir_binary_destroy": (ctypes.c_int, [_vp]),
    "etir_unary_create": (ctypes.c_int, [ctypes.c_char_p, _i64p, ctypes.c_int64, ctypes.c_int32,
                                         ctypes.c_int32, ctypes.POINTER(_vp)]),
    "etir_unary_eval": (ctypes.c_int, [_vp, _vp, _vp]),
    "etir_unary_destroy": (ctypes.c_int, [_vp]),
    "etir_expression_create": (ctypes.c_int, [ctypes.c_char_p, _i64p, ctypes.c_int64, _i64p, ctypes.c_int64,
                                              ctypes.c_int32, ctypes.POINTER(_vp), _vp, ctypes.POINTER(_vp)]),
    "etir_expression_create_ctype": (ctypes.c_int, [ctypes.c_char_p, _i64p, ctypes.c_int64, _i64p, ctypes.c_int64,
                                                    ctypes.c_int32, ctypes.c_int32, ctypes.POINTER(_vp), _vp,
                                                    ctypes.POINTER(_vp)]),
    "etir_expression_eval": (ctypes.c_int, [_vp]),
    "etir_expression_eval_async": (ctypes.c_int, [_vp]),
    "etir_expression_eval_graph": (ctypes.c_int, [_vp]),
    "etir_expression_eval_graph_async": (ctypes.c_int, [_vp]),
    "etir_expression_num_ops": (ctypes.c_int64, [_vp]),
    "etir_expression_store_and_lock_data": (ctypes.c_int, [_vp, ctypes.c_int64]),
    "etir_expression_unlock_data": (ctypes.c_int, [_vp, ctypes.c_int64]),
    "etir_expression_arena_bytes": (ctypes.c_int64, [_vp]),
    "etir_expression_destroy": (ctypes.c_int, [_vp]),
    "etir_tree_count_nodes": (ctypes.c_int64, [ctypes.c_char_p]),
    "etir_tree_create": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int32, ctypes.POINTER(_vp),
                                        _vp, ctypes.POINTER(_vp)]),
    "etir_tree_eval": (ctypes.c_int, [_vp]),
    "etir_tree_num_ops": (ctypes.c_int64, [_vp]),
    "etir_tree_destroy": (ctypes.c_int, [_vp]),
    "etir_nodes_create": (ctypes.c_int, [ctypes.c_int64, _i64p, _i64p, ctypes.c_int64, _i64p, _i64p, _vp,
                                         ctypes.POINTER(_vp)]),
    "etir_nodes_add_leaf": (ctypes.c_int, [_vp, ctypes.c_int64, _i64p, ctypes.c_int32, _vp, _i64p]),
    "etir_nodes_add_binary": (ctypes.c_int, [_vp, ctypes.c_int64, _i64p, ctypes.c_int32, _vp, _vp,
                                             ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int64,
                                             ctypes.c_int64, _i64p]),
    "etir_nodes_compile": (ctypes.c_int, [_vp, ctypes.c_int64]),
    "etir_nodes_store_and_lock_data": (ctypes.c_int, [_vp, ctypes.c_int64]),
    "etir_nodes_unlock_data": (ctypes.c_int, [_vp, ctypes.c_int64]),
    "etir_nodes_eval": (ctypes.c_int, [_vp]),
    "etir_nodes_eval_async": (ctypes.c_int, [_vp]),
    "etir_nodes_eval_graph": (ctypes.c_int, [_vp]),
    "etir_nodes_eval_graph_async": (ctypes.c_int, [_vp]),
    "etir_nodes_num_ops": (ctypes.c_int64, [_vp]),
    "etir_nodes_destroy": (ctypes.c_int, [_vp]),
}


def host_lib():
    """Loads libeinsum_ir.so (in-tree); raises if it has not been built."""
    global _lib_host
    if _lib_host is None:
        _lib.hip_lib()   # dependency first (same directory)
        if not os.path.exists(_lib.LIB_HOST_PATH):
            raise ImportError(f"{_lib.LIB_HOST_PATH} is missing: run __graft_entry__.build() first")
        lib = ctypes.CDLL(_lib.LIB_HOST_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib_host = lib
    return _lib_host


def _check(code):
    if code != _lib.SUCCESS:
        msg = _lib.hip_lib().etir_hip_last_error()
        raise _lib.EinsumIrError(code, msg.decode() if msg else "")


def _ptr(x):
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


def _stream(s):
    if s is None:
        return None
    return s if isinstance(s, int) else s.cuda_stream


def dim_names(expr):
    """Dimension names of an expression sorted into id order (the rule of
    EinsumExpressionAscii::parse_dim_ids: numeric names numerically, others
    lexicographically)."""
    expr = expr.replace(" ", "")
    if expr.startswith("["):
        names = set(n for n in re.split(r"[\[\],]|->", expr) if n)
    else:
        names = set(c for c in expr if c not in ",->")

    def key(n):
        try:
            return (0, int(n), "")
        except ValueError:
            return (1, 0, n)
    return sorted(names, key=key)


def sizes_in_id_order(expr, sizes):
    """Sizes list in ascending dim-id order from a {name: size} dict (or a list)."""
    if isinstance(sizes, dict):
        return [sizes[n] for n in dim_names(expr)]
    return list(sizes)


class _Handle:
    _destroy = None

    def __init__(self):
        self._h = ctypes.c_void_p()

    def close(self):
        if self._h:
            getattr(host_lib(), self._destroy)(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Binary(_Handle):
    """BinaryContractionHip built from an einsum string (BinaryContraction API)."""
    _destroy = "etir_binary_destroy"

    def __init__(self, expr, sizes, dtype_left=_lib.FP32, dtype_right=_lib.FP32, dtype_comp=_lib.FP32,
                 dtype_out=_lib.FP32, ktype_first_touch=_lib.ZERO, ktype_main=_lib.MADD,
                 ktype_last_touch=_lib.UNDEFINED_KTYPE, aux_outer_sizes=None):
        super().__init__()
        s = sizes_in_id_order(expr, sizes)
        aux = _lib.i64_array(sizes_in_id_order(expr, aux_outer_sizes)) if aux_outer_sizes is not None else None
        _check(host_lib().etir_binary_create(expr.encode(), _lib.i64_array(s), len(s), aux,
                                             dtype_left, dtype_right, dtype_comp, dtype_out,
                                             ktype_first_touch, ktype_main, ktype_last_touch,
                                             ctypes.byref(self._h)))

    def contract(self, left, right, out, aux=None):
        _check(host_lib().etir_binary_contract(self._h, _ptr(left), _ptr(right), _ptr(aux), _ptr(out)))

    def num_ops(self):
        return int(host_lib().etir_binary_num_ops(self._h))

    def sizes_cmnk(self):
        nd = (ctypes.c_int64 * 4)()
        sz = (ctypes.c_int64 * 4)()
        _check(host_lib().etir_binary_sizes(self._h, nd, sz))
        return list(nd), list(sz)


class Unary(_Handle):
    """UnaryHip built from "abcd->dbca" (Unary API)."""
    _destroy = "etir_unary_destroy"

    def __init__(self, expr, sizes, dtype=_lib.FP32, ktype=_lib.COPY):
        super().__init__()
        s = sizes_in_id_order(expr, sizes)
        _check(host_lib().etir_unary_create(expr.encode(), _lib.i64_array(s), len(s), dtype, ktype,
                                            ctypes.byref(self._h)))

    def eval(self, inp, out):
        _check(host_lib().etir_unary_eval(self._h, _ptr(inp), _ptr(out)))


# complex_t (reference src/constants.h:54-59)
REAL_ONLY, BATCH_INNER, BATCH_OUTER = 0, 1, 2


class Expression(_Handle):
    """EinsumExpression: einsum string + contraction path, evaluated on the GPU.

    tensors: the input tensors followed by the output tensor (device memory).
    path: flat list or list of pairs in opt_einsum's standard form."""
    _destroy = "etir_expression_destroy"

    def __init__(self, expr, sizes, path, tensors, dtype=_lib.FP32, stream=None, ctype=REAL_ONLY):
        super().__init__()
        s = sizes_in_id_order(expr, sizes)
        flat = []
        for p in path:
            flat.extend(p if isinstance(p, (tuple, list)) else [p])
        self._tensors = list(tensors)   # keep the buffers alive
        ptrs = (ctypes.c_void_p * len(self._tensors))(*[_ptr(t) for t in self._tensors])
        _check(host_lib().etir_expression_create_ctype(expr.encode(), _lib.i64_array(s), len(s),
                                                       _lib.i64_array(flat), len(flat), ctype, dtype, ptrs,
                                                       _stream(stream), ctypes.byref(self._h)))

    def eval(self):
        _check(host_lib().etir_expression_eval(self._h))

    def eval_async(self):
        _check(host_lib().etir_expression_eval_async(self._h))

    def eval_graph(self):
        """eval() as the replay of a recorded HIP graph (needs a stream other
        than the null stream at construction); waits for the replay."""
        _check(host_lib().etir_expression_eval_graph(self._h))

    def eval_graph_async(self):
        _check(host_lib().etir_expression_eval_graph_async(self._h))

    def num_ops(self):
        return int(host_lib().etir_expression_num_ops(self._h))

    def store_and_lock_data(self, tensor_id):
        _check(host_lib().etir_expression_store_and_lock_data(self._h, tensor_id))

    def unlock_data(self, tensor_id):
        _check(host_lib().etir_expression_unlock_data(self._h, tensor_id))

    def arena_bytes(self):
        return int(host_lib().etir_expression_arena_bytes(self._h))


class Tree(_Handle):
    """EinsumTree from the bracketed tree format; tensors: one per node in
    post-order (None for intermediate nodes)."""
    _destroy = "etir_tree_destroy"

    def __init__(self, tree, dim_sizes, tensors, dtype=_lib.FP32, stream=None):
        super().__init__()
        self._tensors = list(tensors)
        ptrs = (ctypes.c_void_p * len(self._tensors))(*[_ptr(t) for t in self._tensors])
        sizes = ",".join(str(x) for x in dim_sizes) if not isinstance(dim_sizes, str) else dim_sizes
        _check(host_lib().etir_tree_create(tree.encode(), sizes.encode(), dtype, ptrs, _stream(stream),
                                           ctypes.byref(self._h)))

    @staticmethod
    def count_nodes(tree):
        return int(host_lib().etir_tree_count_nodes(tree.encode()))

    def eval(self):
        _check(host_lib().etir_tree_eval(self._h))

    def num_ops(self):
        return int(host_lib().etir_tree_num_ops(self._h))


class Nodes(_Handle):
    """EinsumNode tree built node by node (the reference's bench_mlp way).

    sizes: {dim_id: size}; aux_sizes: {dim_id: outer size of the auxiliary
    tensors} (1 for the dims a bias broadcasts over).  add_leaf/add_binary
    return node ids; tensors are device tensors (or raw pointers), None for
    intermediates."""
    _destroy = "etir_nodes_destroy"

    def __init__(self, sizes, aux_sizes=None, stream=None):
        super().__init__()
        ids = sorted(sizes)
        aux = sorted(aux_sizes or {})
        self._keep = []
        _check(host_lib().etir_nodes_create(len(ids), _lib.i64_array(ids), _lib.i64_array([sizes[i] for i in ids]),
                                            len(aux), _lib.i64_array(aux),
                                            _lib.i64_array([aux_sizes[i] for i in aux]) if aux else None,
                                            _stream(stream), ctypes.byref(self._h)))

    def add_leaf(self, dim_ids, tensor, dtype=_lib.FP32):
        node = ctypes.c_int64()
        self._keep.append(tensor)
        _check(host_lib().etir_nodes_add_leaf(self._h, len(dim_ids), _lib.i64_array(dim_ids), dtype, _ptr(tensor),
                                              ctypes.byref(node)))
        return node.value

    def add_binary(self, dim_ids, left, right, tensor=None, aux=None, first=_lib.ZERO, main=_lib.MADD,
                   last=_lib.UNDEFINED_KTYPE, dtype=_lib.FP32):
        node = ctypes.c_int64()
        self._keep.extend([tensor, aux])
        _check(host_lib().etir_nodes_add_binary(self._h, len(dim_ids), _lib.i64_array(dim_ids), dtype, _ptr(aux),
                                                _ptr(tensor), first, main, last, left, right, ctypes.byref(node)))
        return node.value

    def compile(self, root):
        _check(host_lib().etir_nodes_compile(self._h, root))

    def store_and_lock_data(self, node):
        _check(host_lib().etir_nodes_store_and_lock_data(self._h, node))

    def unlock_data(self, node):
        _check(host_lib().etir_nodes_unlock_data(self._h, node))

    def eval(self):
        _check(host_lib().etir_nodes_eval(self._h))

    def eval_async(self):
        _check(host_lib().etir_nodes_eval_async(self._h))

    def eval_graph(self):
        """One evaluation as a replay of a recorded HIP graph (recorded on the
        first call; needs a stream of its own); waits for it."""
        _check(host_lib().etir_nodes_eval_graph(self._h))

    def eval_graph_async(self):
        _check(host_lib().etir_nodes_eval_graph_async(self._h))

    def num_ops(self):
        return int(host_lib().etir_nodes_num_ops(self._h))
