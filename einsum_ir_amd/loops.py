"""Lowering of einsum strings to the loop IR accepted by the C ABI.

Python restatement (for Python callers of the C ABI) of what the reference's
operator classes do before handing loops to a backend:

* dimension typing -- BinaryContraction::dim_types / dim_types_ids
  (reference src/backend/BinaryContraction.cpp:7-221): C = left & right & out,
  M = left & out, N = right & out, K = left & right, I = left only,
  J = right only;
* row-major strides keyed by dimension, 0 for dims of size < 2 --
  BinaryContraction::strides (BinaryContraction.cpp:223-248);
* loop order C, M, N (output order) then K (left order), one loop per
  dimension with the strides of every tensor -- BinaryContractionTpp::compile
  (reference src/backend/BinaryContractionTpp.cpp:46-66);
* the unary path's sizes and input strides in output order --
  Unary::compile_base (reference src/backend/Unary.cpp:82-113).

The C++ classes in libeinsum_ir.so do the same for C++ callers.
"""
from ._lib import DIM_C, DIM_M, DIM_N, DIM_K, DIM_I, DIM_J


def _split(expr):
    expr = expr.replace(" ", "")
    lhs, out = expr.split("->")
    ins = lhs.split(",")
    return ins, out


def dim_types(left, right, out):
    """Dimension types of the output, left and right tensors (lists of names)."""
    def typ(d, in_l, in_r, in_o):
        if in_l and in_r and in_o:
            return DIM_C
        if in_l and in_o:
            return DIM_M
        if in_r and in_o:
            return DIM_N
        if in_l and in_r:
            return DIM_K
        if in_l:
            return DIM_I
        if in_r:
            return DIM_J
        return None
    sl, sr, so = set(left), set(right), set(out)
    return {d: typ(d, d in sl, d in sr, d in so) for d in list(left) + list(right) + list(out)}


def row_major_strides(dims, sizes):
    """Row-major element strides of a tensor; dims of size < 2 get stride 0."""
    strides = {}
    acc = 1
    for d in reversed(list(dims)):
        strides[d] = acc if sizes[d] >= 2 else 0
        acc *= sizes[d]
    return strides


def binary_loops(expr, sizes, sizes_outer_left=None, sizes_outer_right=None,
                 sizes_outer_out=None, sizes_outer_aux=None):
    """Loop IR of a binary contraction ``"ab,bc->ac"``.

    sizes maps dimension names to (inner) sizes; the optional outer-size maps
    describe tensors that are views into larger buffers (the reference's
    outer sizes).  Returns a dict with dim_types, sizes and the four stride
    lists, in the reference's loop order (C, M, N, K)."""
    (left, right), out = _split(expr)
    types = dim_types(left, right, out)
    sl = row_major_strides(left, sizes_outer_left or sizes)
    sr = row_major_strides(right, sizes_outer_right or sizes)
    so = row_major_strides(out, sizes_outer_out or sizes)
    sa = row_major_strides(out, sizes_outer_aux) if sizes_outer_aux else so
    order = ([d for d in out if types[d] == DIM_C] + [d for d in out if types[d] == DIM_M]
             + [d for d in out if types[d] == DIM_N] + [d for d in left if types[d] == DIM_K])
    return {
        "dims": order,
        "dim_types": [types[d] for d in order],
        "sizes": [sizes[d] for d in order],
        "strides_left": [sl.get(d, 0) for d in order],
        "strides_right": [sr.get(d, 0) for d in order],
        "strides_out": [so.get(d, 0) for d in order],
        "strides_out_aux": [sa.get(d, 0) for d in order],
    }


def unary_dims(expr, sizes):
    """Sizes, input strides (reordered to output order) and output strides of a
    permutation ``"abcd->dbca"`` with row-major tensors."""
    (inp,), out = _split(expr)
    # Unary::strides uses the plain row-major product (no zero for size 1)
    si, acc = {}, 1
    for d in reversed(inp):
        si[d] = acc
        acc *= sizes[d]
    so, acc = {}, 1
    for d in reversed(out):
        so[d] = acc
        acc *= sizes[d]
    return {
        "dims": list(out),
        "sizes": [sizes[d] for d in out],
        "strides_in": [si[d] for d in out],
        "strides_out": [so[d] for d in out],
    }
