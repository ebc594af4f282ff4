"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

The reference ships no float fixtures (its float tests compare against ATen
on unseeded random data), so every oracle function is pinned against
library routines and closed forms chosen so that a dropped term, a wrong
index or a transposed operand fails at least one test:
  - numpy.einsum in float64 on random multi-mode layouts,
  - right operand = ones -> row sums (the reference's bench_binary input,
    reference src/bench_binary.cpp:57-59), identity operands,
  - every first/last-touch kernel against its closed form, including the
    broadcast auxiliary tensors of the reference's COPY tests
    (reference src/backend/BinaryContractionTpp.test.torch.cpp:77-367),
  - the reference lowering's treatment of I/J loops (not iterated),
  - bf16 rounding against hand-computed ties and torch.bfloat16,
  - permutations against numpy.transpose, bit for bit.
"""
import itertools

import numpy as np
import pytest

from tests.helpers import parse_binary, tensor_numel, rel_frobenius, loops_for

EXPRS = [
    ("ab,bc->ac", dict(a=5, b=7, c=3)),
    ("abkl,cdkl->abcd", dict(a=3, b=2, c=4, d=3, k=5, l=2)),
    ("zakm,zbkn->zabmn", dict(z=2, a=3, k=4, m=5, b=2, n=3)),
    ("kmc,nkc->nmc", dict(k=6, m=4, c=3, n=5)),
    ("bi,ih->bh", dict(b=4, i=9, h=6)),
    ("dace,bdc->abe", dict(a=2, b=3, c=4, d=2, e=3)),
    ("ba,cb->ac", dict(a=7, b=1, c=4)),   # size-1 K dim (stride 0)
]


def _run(oracle, expr, sizes, rng, first=0, last=99, aux_outer=None, with_aux=False):
    left, right, out = parse_binary(expr)
    loops = loops_for(expr, sizes, sizes_outer_aux=aux_outer)
    a = rng.uniform(-1, 1, tensor_numel(left, sizes))
    b = rng.uniform(-1, 1, tensor_numel(right, sizes))
    o0 = rng.uniform(-1, 1, tensor_numel(out, sizes))
    aux_sizes = aux_outer or sizes
    x = rng.uniform(-1, 1, tensor_numel(out, aux_sizes)) if with_aux else None
    o = o0.copy()
    oracle.contract(loops, a, b, o, aux=x, dtype_left=oracle.FP64, dtype_right=oracle.FP64,
                    dtype_out=oracle.FP64, first_touch=first, last_touch=last)
    shp = lambda dims, s: [s[d] for d in dims]
    ref = np.einsum(expr, a.reshape(shp(left, sizes)), b.reshape(shp(right, sizes)))
    xa = x.reshape(shp(out, aux_sizes)) if with_aux else None
    return o.reshape(shp(out, sizes)), ref, o0.reshape(shp(out, sizes)), xa


@pytest.mark.parametrize("expr,sizes", EXPRS)
def test_contract_matches_numpy_einsum(oracle, expr, sizes):
    rng = np.random.default_rng(1)
    o, ref, _, _ = _run(oracle, expr, sizes, rng)
    np.testing.assert_allclose(o, ref, rtol=1e-12, atol=1e-12)


def test_contract_ones_gives_row_sums(oracle):
    sizes = dict(a=4, b=3, c=5, d=2, k=6, l=3)
    left, right, out = parse_binary("abkl,cdkl->abcd")
    loops = loops_for("abkl,cdkl->abcd", sizes)
    rng = np.random.default_rng(2)
    a = rng.uniform(-1, 1, tensor_numel(left, sizes))
    b = np.ones(tensor_numel(right, sizes))
    o = np.zeros(tensor_numel(out, sizes))
    oracle.contract(loops, a, b, o, dtype_left=1, dtype_right=1, dtype_out=1)
    rs = a.reshape(4, 3, 18).sum(axis=2)
    np.testing.assert_allclose(o.reshape(4, 3, 10), np.repeat(rs[:, :, None], 10, axis=2), rtol=1e-13)


def test_contract_identity(oracle):
    sizes = dict(a=6, b=6, c=6)
    loops = loops_for("ab,bc->ac", sizes)
    rng = np.random.default_rng(3)
    a = rng.uniform(-1, 1, 36)
    o = np.zeros(36)
    oracle.contract(loops, a, np.eye(6).ravel(), o, dtype_left=1, dtype_right=1, dtype_out=1)
    np.testing.assert_array_equal(o, a)
    o = np.zeros(36)
    oracle.contract(loops, np.eye(6).ravel(), a, o, dtype_left=1, dtype_right=1, dtype_out=1)
    np.testing.assert_array_equal(o, a)


@pytest.mark.parametrize("first,last", [(3, 99), (2, 99), (99, 99), (0, 1), (3, 1), (0, 2), (2, 2)])
def test_touch_kernels_closed_form(oracle, first, last):
    rng = np.random.default_rng(4)
    o, ref, o0, x = _run(oracle, "abkl,cdkl->abcd", dict(a=3, b=2, c=4, d=3, k=5, l=2), rng,
                         first=first, last=last, with_aux=True)
    v = ref.copy()
    if first == 3:
        v = x + v
    elif first == 2:
        v = o0 + x + v
    elif first == 99:
        v = o0 + v
    if last == 1:
        v = np.maximum(v, 0.0)
    elif last == 2:
        v = v + x
    np.testing.assert_allclose(o, v, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("bcast", ["full", "row", "col", "scalar"])
def test_copy_broadcast_aux(oracle, bcast):
    # ab,bc->ac with aux of outer sizes (a or 1, c or 1): stride 0 broadcasts
    sizes = dict(a=5, b=4, c=3)
    aux_outer = {"full": dict(a=5, c=3), "row": dict(a=1, c=3),
                 "col": dict(a=5, c=1), "scalar": dict(a=1, c=1)}[bcast]
    aux_outer = dict(aux_outer, b=4)
    rng = np.random.default_rng(5)
    o, ref, _, x = _run(oracle, "ab,bc->ac", sizes, rng, first=3, aux_outer=aux_outer, with_aux=True)
    np.testing.assert_allclose(o, ref + x, rtol=1e-12, atol=1e-12)


def test_ij_loops_not_iterated(oracle):
    # 'i' only in left, 'j' only in right: the reference lowering emits C/M/N/K loops
    # only, so the I/J index stays 0 (reference BinaryContractionTpp.cpp:46-66)
    sizes = dict(i=3, a=4, b=5, j=2, c=6)
    left, right, out = "iab", "bjc", "ac"
    from einsum_ir_amd import dim_types, row_major_strides
    t = dim_types(left, right, out)
    sl, sr, so = (row_major_strides(x, sizes) for x in (left, right, out))
    dims = ["a", "c", "b", "i", "j"]
    loops = dict(dim_types=[t[d] for d in dims], sizes=[sizes[d] for d in dims],
                 strides_left=[sl.get(d, 0) for d in dims], strides_right=[sr.get(d, 0) for d in dims],
                 strides_out=[so.get(d, 0) for d in dims])
    rng = np.random.default_rng(6)
    a = rng.uniform(-1, 1, 60)
    b = rng.uniform(-1, 1, 60)
    o = np.zeros(24)
    oracle.contract(loops, a, b, o, dtype_left=1, dtype_right=1, dtype_out=1)
    ref = a.reshape(3, 4, 5)[0] @ b.reshape(5, 2, 6)[:, 0, :]
    np.testing.assert_allclose(o.reshape(4, 6), ref, rtol=1e-12)


def test_fp32_and_bf16_inputs(oracle):
    sizes = dict(a=8, b=16, c=4)
    loops = loops_for("ab,bc->ac", sizes)
    rng = np.random.default_rng(7)
    a = rng.uniform(-1, 1, 128).astype(np.float32)
    b = rng.uniform(-1, 1, 64).astype(np.float32)
    o = np.zeros(32, dtype=np.float32)
    oracle.contract(loops, a, b, o)
    ref = a.astype(np.float64).reshape(8, 16) @ b.astype(np.float64).reshape(16, 4)
    assert rel_frobenius(ref, o) < 1e-7
    ab, bb = oracle.f32_to_bf16(a), oracle.f32_to_bf16(b)
    o = np.zeros(32, dtype=np.float32)
    oracle.contract(loops, ab, bb, o, dtype_left=2, dtype_right=2)
    ref = (oracle.bf16_to_f32(ab).astype(np.float64).reshape(8, 16)
           @ oracle.bf16_to_f32(bb).astype(np.float64).reshape(16, 4))
    assert rel_frobenius(ref, o) < 1e-7


def test_bf16_rounding_ties():
    from oracle import py_oracle as po
    one = 1.0
    vals = np.array([one, one + 2.0 ** -8, one + 3 * 2.0 ** -8, one + 2.0 ** -8 + 2.0 ** -20,
                     -2.5, 0.0, -0.0, np.inf, -np.inf], dtype=np.float32)
    bits = po.f32_to_bf16(vals)
    assert [int(x) for x in bits] == [0x3F80, 0x3F80, 0x3F82, 0x3F81, 0xC020, 0x0000, 0x8000,
                                      0x7F80, 0xFF80]
    nan = po.f32_to_bf16(np.array([np.nan], dtype=np.float32))
    assert (int(nan[0]) & 0x7F80) == 0x7F80 and (int(nan[0]) & 0x7F) != 0
    np.testing.assert_array_equal(po.bf16_to_f32(bits[:5]), np.array([1.0, 1.0, 1.0 + 2 ** -6,
                                                                     1.0 + 2 ** -7, -2.5], np.float32))


def test_bf16_rounding_matches_torch():
    torch = pytest.importorskip("torch")
    from oracle import py_oracle as po
    rng = np.random.default_rng(8)
    x = (rng.standard_normal(100000) * rng.choice([1e-3, 1.0, 1e3], 100000)).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(po.f32_to_bf16(x), ref)


PERMS = [("abcd->dbca", dict(a=5, b=3, c=4, d=6)), ("ab->ba", dict(a=7, b=9)),
         ("abc->abc", dict(a=2, b=3, c=4)), ("abcde->ecadb", dict(a=2, b=3, c=2, d=4, e=3))]


@pytest.mark.parametrize("expr,sizes", PERMS)
@pytest.mark.parametrize("dtype", [0, 1, 2])
def test_permute_matches_numpy(oracle, expr, sizes, dtype):
    from einsum_ir_amd import unary_dims
    u = unary_dims(expr, sizes)
    inp_dims, out_dims = expr.split("->")
    rng = np.random.default_rng(9)
    n = tensor_numel(inp_dims, sizes)
    npdt = {0: np.float32, 1: np.float64, 2: np.uint16}[dtype]
    x = rng.integers(0, 2 ** 15, n).astype(npdt) if dtype == 2 else rng.uniform(-1, 1, n).astype(npdt)
    o = np.zeros(n, dtype=npdt)
    oracle.permute(u["sizes"], u["strides_in"], u["strides_out"], x, o, dtype=dtype, ktype=oracle.COPY)
    ref = np.transpose(x.reshape([sizes[d] for d in inp_dims]), [inp_dims.index(d) for d in out_dims])
    np.testing.assert_array_equal(o, ref.ravel())
    # ADD adds the permuted input, ZERO clears
    o2 = o.copy()
    if dtype != 2:
        oracle.permute(u["sizes"], u["strides_in"], u["strides_out"], x, o2, dtype=dtype, ktype=oracle.ADD)
        np.testing.assert_array_equal(o2, ref.ravel() * 2)
    oracle.permute(u["sizes"], u["strides_in"], u["strides_out"], x, o2, dtype=dtype, ktype=oracle.ZERO)
    assert not np.any(o2)


@pytest.mark.parametrize("expr,sizes", EXPRS[:6])
@pytest.mark.parametrize("first,last", [(0, 99), (3, 1), (99, 2)])
def test_blocked_baseline_matches_exact(oracle, expr, sizes, first, last):
    left, right, out = parse_binary(expr)
    loops = loops_for(expr, sizes)
    rng = np.random.default_rng(10)
    a = rng.uniform(-1, 1, tensor_numel(left, sizes)).astype(np.float32)
    b = rng.uniform(-1, 1, tensor_numel(right, sizes)).astype(np.float32)
    x = rng.uniform(-1, 1, tensor_numel(out, sizes)).astype(np.float32)
    o0 = rng.uniform(-1, 1, tensor_numel(out, sizes)).astype(np.float32)
    o1, o2 = o0.copy(), o0.copy()
    oracle.contract(loops, a, b, o1, aux=x, first_touch=first, last_touch=last)
    oracle.contract_blocked(loops, a, b, o2, aux=x, first_touch=first, last_touch=last, num_threads=2)
    assert rel_frobenius(o1, o2) < 1e-6


def test_contract_path_matches_numpy(oracle):
    # the tree oracle along a path equals numpy.einsum in float64
    expr = "da,dce,bec->abc"
    sizes = dict(a=3, b=4, c=5, d=2, e=3)
    rng = np.random.default_rng(11)
    ins = expr.split("->")[0].split(",")
    arrs = [rng.uniform(-1, 1, tensor_numel(t, sizes)) for t in ins]
    got = oracle.contract_path(expr, sizes, [(1, 2), (0, 1)], arrs)
    ref = np.einsum(expr, *[a.reshape([sizes[d] for d in t]) for a, t in zip(arrs, ins)])
    np.testing.assert_allclose(got, ref.ravel(), rtol=1e-12, atol=1e-12)


def test_contract_path_bf16_rounding(oracle):
    # round_bf16 rounds every step's result: equal to numpy.einsum steps with
    # torch's own bfloat16 conversion (round to nearest even) in between
    torch = pytest.importorskip("torch")
    expr = "da,dce,bec->abc"
    sizes = dict(a=3, b=4, c=5, d=2, e=3)
    rng = np.random.default_rng(12)
    ins = expr.split("->")[0].split(",")
    arrs = [rng.uniform(-1, 1, tensor_numel(t, sizes)) for t in ins]
    got = oracle.contract_path(expr, sizes, [(1, 2), (0, 1)], arrs, round_bf16=True)

    def rnd(x):
        return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).bfloat16().float().double().numpy()

    sh = lambda a, t: a.reshape([sizes[d] for d in t])
    # step 1: dce,bec -> intermediate dims {b, c, d} in ascending name order
    t1 = rnd(np.einsum("dce,bec->bcd", sh(arrs[1], "dce"), sh(arrs[2], "bec")))
    ref = rnd(np.einsum("da,bcd->abc", sh(arrs[0], "da"), t1))
    assert np.array_equal(got, ref.ravel())
    # without rounding the same path differs from the rounded one
    plain = oracle.contract_path(expr, sizes, [(1, 2), (0, 1)], arrs)
    assert not np.array_equal(plain, got)


@pytest.mark.parametrize("expr,sizes", [
    ("abcd->dbca", dict(a=7, b=5, c=9, d=70)),
    ("abc->cba", dict(a=65, b=3, c=130)),
    ("ab->ba", dict(a=129, b=64)),
    ("abcd->acdb", dict(a=3, b=66, c=4, d=5)),
])
def test_permute_blocked_matches_permute(oracle, expr, sizes):
    # the blocked CPU baseline equals the reference-semantics permutation bit for bit
    from einsum_ir_amd import unary_dims
    u = unary_dims(expr, sizes)
    n = int(np.prod(list(sizes.values())))
    x = np.random.default_rng(5).uniform(-1, 1, n).astype(np.float32)
    y1, y2 = np.zeros_like(x), np.full_like(x, np.nan)
    oracle.permute(u["sizes"], u["strides_in"], u["strides_out"], x, y1)
    assert oracle.permute_blocked(u["sizes"], u["strides_in"], u["strides_out"], x, y2)
    assert np.array_equal(y1, y2)


def test_permute_blocked_declines_same_unit_dim(oracle):
    from einsum_ir_amd import unary_dims
    u = unary_dims("abc->bac", dict(a=4, b=5, c=6))
    x = np.zeros(120, np.float32)
    assert not oracle.permute_blocked(u["sizes"], u["strides_in"], u["strides_out"], x, x.copy())
