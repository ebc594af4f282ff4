"""GPU parity of the permutation path (etir_hip_permute_*) -- bit-exact.

Mirrors the reference's unary tests (reference src/backend/UnaryTpp.test.torch.cpp,
src/basic/unary/UnaryBackendTpp.test.torch.cpp: transposes of up to 9 dims
checked with at::equal) with seeded inputs and the CPU oracle as checker.
"""
import re

import numpy as np
import pytest

import einsum_ir_amd as eir
from tests.helpers import tensor_numel

pytestmark = pytest.mark.gpu

NPDT = {eir.FP32: np.float32, eir.FP64: np.float64, eir.BF16: np.uint16}


def _to_dev(torch, x):
    if x.dtype == np.uint16:
        return torch.from_numpy(x.view(np.int16)).cuda()
    return torch.from_numpy(x).cuda()


def _from_dev(t, npdt):
    a = t.cpu().numpy()
    return a.view(np.uint16) if npdt == np.uint16 else a


def _inputs(rng, n, dtype):
    if dtype == eir.BF16:
        return rng.integers(0, 2 ** 16, n, dtype=np.uint64).astype(np.uint16)
    return rng.uniform(-1, 1, n).astype(NPDT[dtype])


def _check(torch, oracle, expr, sizes, dtype=eir.FP32, ktype=eir.COPY, seed=0):
    u = eir.unary_dims(expr, sizes)
    inp, _ = expr.split("->")
    n = tensor_numel(inp, sizes)
    rng = np.random.default_rng(seed)
    x = _inputs(rng, n, dtype)
    o0 = _inputs(rng, n, dtype) if dtype != eir.BF16 else rng.integers(0, 2 ** 14, n).astype(np.uint16)
    ref = o0.copy()
    oracle.permute(u["sizes"], u["strides_in"], u["strides_out"], x, ref, dtype=dtype, ktype=ktype)
    plan = eir.PermutePlan(u["sizes"], u["strides_in"], u["strides_out"], dtype=dtype, ktype=ktype)
    dx, do = _to_dev(torch, x), _to_dev(torch, o0)
    stream = torch.cuda.current_stream()
    plan.execute(dx, do, stream=stream)
    torch.cuda.synchronize()
    got = _from_dev(do, NPDT[dtype])
    desc = plan.describe()
    plan.close()
    np.testing.assert_array_equal(got.view(np.uint8), ref.view(np.uint8), err_msg=desc)
    return desc


def test_c2_abcd_dbca_64(torch_cuda, oracle):
    """BASELINE config 2 at full size: abcd->dbca, 64^4 fp32, bit-exact."""
    desc = _check(torch_cuda, oracle, "abcd->dbca", dict(a=64, b=64, c=64, d=64), seed=2)
    assert "transpose" in desc


CASES = [
    ("ab->ba", dict(a=64, b=64)),
    ("ab->ba", dict(a=67, b=130)),        # ragged tiles
    ("ab->ba", dict(a=1, b=37)),          # size-1 dim
    ("abc->cba", dict(a=9, b=3, c=70)),
    ("abc->acb", dict(a=5, b=66, c=64)),
    ("abc->abc", dict(a=3, b=5, c=64)),   # pure copy, vectorised
    ("abc->abc", dict(a=3, b=5, c=7)),    # pure copy, scalar
    ("abcd->badc", dict(a=2, b=3, c=5, d=7)),
    ("abcde->ecadb", dict(a=4, b=2, c=8, d=2, e=16)),
    ("abcdefghi->ihgfedcba", dict(a=2, b=2, c=3, d=2, e=2, f=3, g=2, h=2, i=4)),  # 9-D
    ("a->a", dict(a=1000)),
]


@pytest.mark.parametrize("expr,sizes", CASES)
@pytest.mark.parametrize("dtype", [eir.FP32, eir.FP64, eir.BF16])
def test_permute_copy(torch_cuda, oracle, expr, sizes, dtype):
    _check(torch_cuda, oracle, expr, sizes, dtype=dtype)


@pytest.mark.parametrize("expr,sizes", [CASES[1], CASES[5], CASES[8]])
@pytest.mark.parametrize("ktype", [eir.ZERO, eir.ADD])
@pytest.mark.parametrize("dtype", [eir.FP32, eir.FP64])
def test_permute_zero_add(torch_cuda, oracle, expr, sizes, ktype, dtype):
    _check(torch_cuda, oracle, expr, sizes, dtype=dtype, ktype=ktype)


@pytest.mark.parametrize("ktype", [eir.COPY, eir.ZERO, eir.ADD])
@pytest.mark.parametrize("offset", [0, 4, 1])
def test_permute_bf16_vector_copy(torch_cuda, oracle, ktype, offset):
    """bf16 copies and fills move 8-element (16-byte) vectors where rows and
    base addresses allow it; a base offset of 4 elements (8-byte aligned) or
    1 element takes the 4-element or the element path.  Bit-exact."""
    torch = torch_cuda
    sizes = [7, 5, 64]                        # output order, innermost unit stride in both
    s_in, s_out = [5 * 72, 72, 1], [5 * 64, 64, 1]
    n_in, n_out = 7 * 5 * 72, 7 * 5 * 64
    rng = np.random.default_rng(40 + offset)
    x = rng.integers(0, 2 ** 16, n_in + offset, dtype=np.uint64).astype(np.uint16)
    o0 = rng.integers(0, 2 ** 14, n_out + offset, dtype=np.uint64).astype(np.uint16)
    ref = o0[offset:].copy()
    oracle.permute(sizes, s_in, s_out, x[offset:].copy(), ref, dtype=eir.BF16, ktype=ktype)
    plan = eir.PermutePlan(sizes, s_in, s_out, dtype=eir.BF16, ktype=ktype)
    dx = torch.from_numpy(x.view(np.int16)).cuda()
    do = torch.from_numpy(o0.view(np.int16)).cuda()
    plan.execute(dx[offset:], do[offset:], stream=torch.cuda.current_stream())
    torch.cuda.synchronize()
    plan.close()
    np.testing.assert_array_equal(do[offset:].cpu().numpy().view(np.uint16), ref)


def test_permute_empty(torch_cuda):
    plan = eir.PermutePlan([0, 4], [4, 1], [4, 1])
    plan.execute(None, None)
    plan.close()


def test_permute_rejects_bad_ktype(torch_cuda):
    with pytest.raises(eir.EinsumIrError) as e:
        eir.PermutePlan([4, 4], [4, 1], [1, 4], ktype=eir.RELU)
    assert e.value.code == eir.INVALID_KTYPE


# both unit-stride dims shorter than a 64-wide tile: tiles over the innermost
# runs of both tensors (shared middle dims, 2-dim runs, ragged edges, 5-D)
TILED_CASES = [
    ("abcd->dbca", dict(a=6, b=64, c=96, d=10)),      # runs (d,c) and (a,c): shared c
    ("abcd->dbca", dict(a=20, b=40, c=48, d=14)),
    ("abcd->dbca", dict(a=5, b=9, c=70, d=13)),       # ragged everywhere
    ("abcd->acdb", dict(a=7, b=13, c=11, d=5)),
    ("abcde->bdaec", dict(a=12, b=9, c=9, d=12, e=16)),
    ("abcde->bdaec", dict(a=3, b=5, c=6, d=7, e=4)),    # many short dims
    ("abc->cba", dict(a=40, b=2, c=20)),               # runs of two dims each
    ("abcd->acdb", dict(a=6, b=8, c=10, d=150)),       # one long unit dim, one of 8
    ("abc->cba", dict(a=4, b=100, c=130)),             # one long unit dim, one of 4
    ("abc->cba", dict(a=3, b=70, c=300)),              # ... of 3 (no 16-byte entries)
]


@pytest.mark.parametrize("expr,sizes", TILED_CASES)
@pytest.mark.parametrize("dtype", [eir.FP32, eir.FP64, eir.BF16])
def test_permute_tiled(torch_cuda, oracle, expr, sizes, dtype):
    desc = _check(torch_cuda, oracle, expr, sizes, dtype=dtype, seed=len(expr))
    # bf16's REG4 limits are twice as long in elements (same bytes)
    assert "tiled" in desc or (dtype == eir.BF16 and "reg4" in desc), desc


@pytest.mark.parametrize("expr,sizes", [TILED_CASES[0], TILED_CASES[2], TILED_CASES[6]])
def test_permute_tiled_add(torch_cuda, oracle, expr, sizes):
    _check(torch_cuda, oracle, expr, sizes, dtype=eir.FP32, ktype=eir.ADD)


# transposes whose unit-stride dims are a short one (<= 32) and a long one:
# 128 x 32 or 32 x 128 tiles (a 64 x 64 tile would be half empty)
TR_SHAPE_CASES = [
    ("abcd->dcba", dict(a=20, b=3, c=5, d=200), "tile=128x32"),
    ("abcd->dcba", dict(a=200, b=3, c=5, d=20), "tile=32x128"),
    ("abc->cba", dict(a=31, b=6, c=130), "tile=128x32"),       # ragged: 31 of 32, 130 of 256
    ("abc->cba", dict(a=129, b=4, c=29), "tile=32x128"),
]


@pytest.mark.parametrize("expr,sizes,tile", TR_SHAPE_CASES)
@pytest.mark.parametrize("dtype", [eir.FP32, eir.FP64])
@pytest.mark.parametrize("ktype", [eir.COPY, eir.ADD])
def test_permute_transpose_shapes(torch_cuda, oracle, expr, sizes, tile, dtype, ktype):
    desc = _check(torch_cuda, oracle, expr, sizes, dtype=dtype, ktype=ktype, seed=sizes["a"] + int(ktype))
    assert "transpose" in desc and tile in desc, desc


# bf16 transposes with 16-byte reads (input rows in groups of 8 elements,
# output rows in groups of 4): 128 x 64 tiles, or 128 x 32 where those fill
# more of their padded grid; ragged extents on both sides.  An output
# unit-stride dim that is not a multiple of 64 is folded with the output's
# next dim when that one continues the output's run (fold=o1xo2, 128 x 64)
TR16_CASES = [
    # o = c (36) folded with a (36): 1296-element o rows
    ("abcd->bdac", dict(a=36, b=5, c=36, d=512), "tile=128x64 v16 fold=36x36"),
    # o = c (72) folded with a (7): 504 o rows
    ("abcd->bdac", dict(a=7, b=3, c=72, d=256), "tile=128x64 v16 fold=72x7"),
    # o = a (64): no fold; i = 200: 200 of 256
    ("abcd->dbca", dict(a=64, b=3, c=5, d=200), "tile=128x64 v16"),
    # o = a (100) folded with b (3)
    ("abc->cba", dict(a=100, b=3, c=136), "tile=128x64 v16 fold=100x3"),
    # o = c (44) folded with a (7), ragged on both sides (i = 200)
    ("abcd->bdac", dict(a=7, b=3, c=44, d=200), "fold=44x7"),
    # o = a (40) folded with b (9), c a batch dim
    ("abcd->dcba", dict(a=40, b=9, c=5, d=136), "fold=40x9"),
    # o = a (24, above 16): the folded transpose rather than register blocks
    ("abcd->dcba", dict(a=24, b=32, c=5, d=128), "tile=128x64 v16 fold=24x32"),
    # no next output dim continues o's run (the input's unit dim d follows o):
    # 128 x 32 where it fills more of its grid
    ("abc->bca", dict(a=72, b=6, c=256), "tile=128x32 v16"),
]


@pytest.mark.parametrize("expr,sizes,tile", TR16_CASES)
@pytest.mark.parametrize("ktype", [eir.COPY, eir.ADD])
def test_permute_transpose16_bf16(torch_cuda, oracle, expr, sizes, tile, ktype):
    desc = _check(torch_cuda, oracle, expr, sizes, dtype=eir.BF16, ktype=ktype, seed=sizes["a"] + int(ktype))
    assert "transpose" in desc and tile in desc, desc


@pytest.mark.parametrize("offset", [1, 4])
def test_permute_transpose16_unaligned(torch_cuda, oracle, offset):
    """The 16-byte-read bf16 transpose on tensors whose base addresses are
    not 16-byte aligned (offset by 1 or 4 elements): one element per access,
    same result."""
    torch = torch_cuda
    sizes = dict(a=36, b=5, c=36, d=512)
    u = eir.unary_dims("abcd->bdac", sizes)
    n = 36 * 5 * 36 * 512
    rng = np.random.default_rng(70 + offset)
    x = rng.integers(0, 2 ** 16, n + offset, dtype=np.uint64).astype(np.uint16)
    o0 = rng.integers(0, 2 ** 14, n + offset, dtype=np.uint64).astype(np.uint16)
    ref = o0[offset:].copy()
    oracle.permute(u["sizes"], u["strides_in"], u["strides_out"], x[offset:].copy(), ref, dtype=eir.BF16)
    plan = eir.PermutePlan(u["sizes"], u["strides_in"], u["strides_out"], dtype=eir.BF16)
    assert "v16 fold=36x36" in plan.describe(), plan.describe()
    dx, do = _to_dev(torch, x), _to_dev(torch, o0)
    plan.execute(dx[offset:], do[offset:], stream=torch.cuda.current_stream())
    torch.cuda.synchronize()
    plan.close()
    np.testing.assert_array_equal(do[offset:].cpu().numpy().view(np.uint16), ref)


# a unit-stride dim shared by both tensors with short rows: whole rows
# through LDS (ROWS), runs of the input's and the output's next dims
ROWS_CASES = [
    ("abcd->cabd", dict(a=6, b=5, c=70, d=36)),        # 144-byte fp32 rows, ragged tiles
    ("abcd->cabd", dict(a=3, b=7, c=9, d=5)),          # 5-element rows: one-element chunks (fp32)
    ("abc->bac", dict(a=37, b=300, c=12)),             # 3 chunks per row, ragged both ways
    ("abc->bac", dict(a=300, b=2, c=12)),              # input runs of 2 rows: many runs per thread step
    ("abcde->dbcae", dict(a=3, b=4, c=5, d=33, e=8)),  # batch dims b, c
    ("abcd->cabd", dict(a=2, b=1, c=3000, d=4)),       # 16-byte rows, one long dim
]


@pytest.mark.parametrize("expr,sizes", ROWS_CASES)
@pytest.mark.parametrize("dtype", [eir.FP32, eir.FP64, eir.BF16])
@pytest.mark.parametrize("ktype", [eir.COPY, eir.ADD])
def test_permute_rows(torch_cuda, oracle, expr, sizes, dtype, ktype):
    desc = _check(torch_cuda, oracle, expr, sizes, dtype=dtype, ktype=ktype, seed=len(expr) + int(ktype))
    rowb = sizes[expr.split("->")[0][-1]] * {eir.FP32: 4, eir.FP64: 8, eir.BF16: 2}[dtype]
    # rows of 16 to 255 bytes (bf16: 127) take ROWS; shorter ones the tiled
    # kernel, longer ones the vector copy
    assert ("rows" in desc) == (16 <= rowb < (128 if dtype == eir.BF16 else 256)), desc


@pytest.mark.parametrize("expr,sizes", [ROWS_CASES[0], ROWS_CASES[2], ROWS_CASES[4]])
def test_permute_rows_switched_off(torch_cuda, oracle, monkeypatch, expr, sizes):
    """With ROWS switched off the tiled kernel moves the same shapes."""
    monkeypatch.setenv("ETIR_PERM_ROWS", "0")
    for dtype in (eir.FP32, eir.BF16):
        desc = _check(torch_cuda, oracle, expr, sizes, dtype=dtype, seed=3)
        assert "tiled" in desc, desc


def test_permute_rows_long(torch_cuda, oracle, monkeypatch):
    """Rows longer than the default limit when the limit is raised: 600-byte
    rows, more chunks per tile than one pass of the threads covers."""
    monkeypatch.setenv("ETIR_PERM_ROWS_MAX_BYTES", "100000")
    for dtype in (eir.FP32, eir.FP64):
        desc = _check(torch_cuda, oracle, "abcd->cabd", dict(a=3, b=9, c=40, d=150), dtype=dtype, seed=9)
        assert "rows" in desc, desc
        desc = _check(torch_cuda, oracle, "abcd->cabd", dict(a=3, b=9, c=40, d=150), dtype=dtype, ktype=eir.ADD)
        assert "rows" in desc, desc


@pytest.mark.parametrize("dtype,offset", [(eir.FP32, 1), (eir.FP32, 2), (eir.BF16, 1), (eir.BF16, 2),
                                          (eir.BF16, 4), (eir.FP64, 1)])
def test_permute_rows_unaligned(torch_cuda, oracle, dtype, offset):
    """ROWS on tensors whose base addresses are offset by a few elements:
    chunks of one element where the plan's chunk width is not aligned."""
    torch = torch_cuda
    expr, sizes = "abcd->cabd", dict(a=6, b=5, c=70, d=28)
    u = eir.unary_dims(expr, sizes)
    n = 6 * 5 * 70 * 28
    rng = np.random.default_rng(50 + offset)
    x = _inputs(rng, n + offset, dtype)
    o0 = _inputs(rng, n + offset, dtype)
    ref = o0[offset:].copy()
    oracle.permute(u["sizes"], u["strides_in"], u["strides_out"], x[offset:].copy(), ref, dtype=dtype)
    plan = eir.PermutePlan(u["sizes"], u["strides_in"], u["strides_out"], dtype=dtype, ktype=eir.COPY)
    dx, do = _to_dev(torch, x), _to_dev(torch, o0)
    plan.execute(dx[offset:], do[offset:], stream=torch.cuda.current_stream())
    torch.cuda.synchronize()
    desc = plan.describe()
    plan.close()
    assert "rows" in desc, desc
    got = _from_dev(do, NPDT[dtype])[offset:]
    np.testing.assert_array_equal(got.view(np.uint8), ref.view(np.uint8), err_msg=desc)


# both unit-stride dims multiples of 4, the shorter <= 16: 4 x 4 register
# transposes (one input dim whose run continues i, else the output's, else the
# largest, is walked by the lanes; long input unit dims are split first)
REG4_CASES = [
    ("abcd->dbca", dict(a=8, b=64, c=96, d=8)),        # c continues both runs
    ("abcd->dbca", dict(a=16, b=40, c=48, d=16)),
    ("abcd->dbca", dict(a=4, b=33, c=17, d=4)),        # ragged last chunk of c
    ("abcd->adcb", dict(a=12, b=8, c=10, d=64)),       # i=64, o=8: one wave of blocks
    ("abcd->acdb", dict(a=3, b=8, c=5, d=256)),        # i=cd=1280 split into 10 x 128
    ("abcd->acdb", dict(a=2, b=4, c=3, d=512)),        # i=cd=1536 split into 6 x 256
    ("abcde->bdeca", dict(a=4, b=6, c=7, d=5, e=8)),   # 5-D, i=de=40, batch dims around c
    ("abc->cba", dict(a=12, b=1, c=16)),               # no dim beside i and o
    ("abcd->dbca", dict(a=20, b=40, c=48, d=12)),      # 15 blocks a value of c: chunk 17
]


@pytest.mark.parametrize("expr,sizes", REG4_CASES)
@pytest.mark.parametrize("dtype", [eir.FP32, eir.FP64, eir.BF16])
def test_permute_reg4(torch_cuda, oracle, expr, sizes, dtype):
    desc = _check(torch_cuda, oracle, expr, sizes, dtype=dtype, seed=3 + len(expr))
    # bf16 blocks are 8 x 8 (16-byte rows): unit dims that are not multiples
    # of 8 take another kernel (test_permute_reg4_bf16 covers its blocks)
    assert "reg4" in desc or dtype == eir.BF16, desc


# bf16: 8 x 8 blocks (16-byte rows) when both unit dims are multiples of 8,
# else 4 x 4; short dims up to 32, both dims up to 64 when whole lines
BF16_REG4_CASES = [
    ("abcd->dbca", dict(a=8, b=64, c=96, d=8), 8),
    ("abcd->dbca", dict(a=16, b=40, c=48, d=16), 8),
    ("abcd->dbca", dict(a=32, b=5, c=6, d=32), 8),         # 32 x 32: short-dim rule
    ("abcd->dbca", dict(a=64, b=3, c=5, d=64), 8),         # 64 x 64: whole 128-byte lines
    ("abcd->dbca", dict(a=8, b=33, c=17, d=24), 8),        # ragged last chunk of c
    ("abcd->acdb", dict(a=3, b=8, c=5, d=256), 8),         # i = cd = 1280, o = 8
    ("abcd->acdb", dict(a=2, b=16, c=3, d=512), 8),        # i = cd = 1536 split into 6 x 256
    ("abcd->dbca", dict(a=4, b=33, c=17, d=4), 4),         # 4-wide dims: 4 x 4 blocks
    ("abcd->dbca", dict(a=12, b=7, c=9, d=20), 4),
]


@pytest.mark.parametrize("expr,sizes,vb", BF16_REG4_CASES)
@pytest.mark.parametrize("ktype", [eir.COPY, eir.ADD])
def test_permute_reg4_bf16(torch_cuda, oracle, expr, sizes, vb, ktype):
    desc = _check(torch_cuda, oracle, expr, sizes, dtype=eir.BF16, ktype=ktype, seed=16 + len(expr))
    assert "reg4" in desc and f" b={vb} " in desc, desc


def test_permute_reg4_bf16_unaligned(torch_cuda, oracle):
    """bf16 REG4 on tensors whose rows are 8-element multiples but whose
    base address is only 2-byte aligned: the element path, bit-exact."""
    torch = torch_cuda
    expr, sizes, _ = BF16_REG4_CASES[0]
    u = eir.unary_dims(expr, sizes)
    n = 8 * 64 * 96 * 8
    rng = np.random.default_rng(21)
    x = rng.integers(0, 2 ** 16, n + 1, dtype=np.uint64).astype(np.uint16)
    ref = np.zeros(n, dtype=np.uint16)
    oracle.permute(u["sizes"], u["strides_in"], u["strides_out"], x[1:].copy(), ref, dtype=eir.BF16)
    plan = eir.PermutePlan(u["sizes"], u["strides_in"], u["strides_out"], dtype=eir.BF16, ktype=eir.COPY)
    dx = torch.from_numpy(x.view(np.int16)).cuda()
    dout = torch.zeros(n + 1, dtype=torch.int16, device="cuda")
    plan.execute(dx[1:], dout[1:], stream=torch.cuda.current_stream())
    torch.cuda.synchronize()
    desc = plan.describe()
    plan.close()
    assert "reg4" in desc
    np.testing.assert_array_equal(dout[1:].cpu().numpy().view(np.uint16), ref)


@pytest.mark.parametrize("expr,sizes", [REG4_CASES[0], REG4_CASES[2], REG4_CASES[4]])
@pytest.mark.parametrize("dtype", [eir.FP32, eir.FP64])
def test_permute_reg4_add(torch_cuda, oracle, expr, sizes, dtype):
    desc = _check(torch_cuda, oracle, expr, sizes, dtype=dtype, ktype=eir.ADD)
    assert "reg4" in desc


@pytest.mark.parametrize("cpt", ["2", "4"])
def test_permute_reg4_passes(torch_cuda, oracle, monkeypatch, cpt):
    """Two and four passes of 256 threads over c (a planner option)."""
    monkeypatch.setenv("ETIR_PERM_REG4_CPT", cpt)
    for expr, sizes in REG4_CASES[:3]:
        desc = _check(torch_cuda, oracle, expr, sizes, seed=int(cpt))
        assert f"t=256x{cpt}" in desc, desc


def test_permute_reg4_passes_beyond_the_lds_limit(torch_cuda, oracle, monkeypatch):
    """A pass count whose LDS tile would exceed 64 KiB (bf16 acdb, a 128-wide
    input run: four passes would need about 130 KiB) is not taken: one pass,
    same bytes."""
    monkeypatch.setenv("ETIR_PERM_REG4_CPT", "4")
    desc = _check(torch_cuda, oracle, "abcd->acdb", dict(a=8, b=16, c=64, d=128), dtype=eir.BF16, seed=44)
    assert "reg4" in desc and re.search(r"t=\d+x1\b", desc), desc


@pytest.mark.parametrize("threads", ["64", "128", "256", "512"])
def test_permute_reg4_workgroup_sizes(torch_cuda, oracle, monkeypatch, threads):
    """Every workgroup size of the REG4 kernel (a planner option, taken when
    it holds the blocks of one value of c)."""
    monkeypatch.setenv("ETIR_PERM_REG4_THREADS", threads)
    for expr, sizes in REG4_CASES[:4]:
        desc = _check(torch_cuda, oracle, expr, sizes, dtype=eir.FP64, seed=int(threads))
        assert f"t={threads}x1" in desc, desc


@pytest.mark.parametrize("dtype,mode32,mode24", [(eir.FP32, "reg4", "tiled"), (eir.FP64, "reg4", "tiled"),
                                                  (eir.BF16, "reg4", "reg4")])
def test_permute_32_wide_unit_dims(torch_cuda, oracle, dtype, mode32, mode24):
    """Unit-stride dims of 32 on both sides take REG4 when each is a whole
    number of 128-byte lines (fp32, fp64) and the tiled kernel otherwise;
    for bf16 (8 x 8 blocks) 32 elements are a short dim."""
    desc = _check(torch_cuda, oracle, "abcd->dbca", dict(a=32, b=5, c=6, d=32), dtype=dtype, seed=32)
    assert mode32 in desc, desc
    desc = _check(torch_cuda, oracle, "abcd->cbda", dict(a=32, b=3, c=7, d=24), dtype=dtype, seed=24)
    assert mode24 in desc, desc


@pytest.mark.parametrize("dtype", [eir.FP32, eir.FP64, eir.BF16])
@pytest.mark.parametrize("direct", ["0", "1"])
def test_permute_reg4_direct_stores(torch_cuda, oracle, monkeypatch, dtype, direct):
    """Rows stored from registers (no LDS exchange) where the planner takes
    them, and the exchange where it is switched off; COPY and ADD."""
    monkeypatch.setenv("ETIR_PERM_REG4_DIRECT", direct)
    for expr, sizes in [REG4_CASES[0], REG4_CASES[1], REG4_CASES[2]]:
        desc = _check(torch_cuda, oracle, expr, sizes, dtype=dtype, seed=7)
        if "reg4" in desc:
            assert ("direct" in desc) == (direct == "1"), desc
        _check(torch_cuda, oracle, expr, sizes, dtype=dtype, ktype=eir.ADD, seed=8)


@pytest.mark.parametrize("expr,sizes,threads", [
    ("abcd->dbca", dict(a=16, b=4, c=32, d=16), 64),      # 16 blocks of 4 x 4 per value of c
    ("abc->cba", dict(a=128, b=3, c=16), 128),             # 128 blocks
    ("abc->cba", dict(a=256, b=3, c=16), 256),             # 256 blocks
])
def test_permute_reg4_default_workgroup(torch_cuda, oracle, expr, sizes, threads):
    """The default is the smallest workgroup of 64, 128 or 256 threads that
    holds one value of c's blocks."""
    desc = _check(torch_cuda, oracle, expr, sizes, seed=threads)
    assert f"t={threads}x1" in desc, desc


def test_permute_4d_bench_shapes(torch_cuda):
    """The 4-D fp32 shapes timed beside config 2, at full size (16.8-31.9 M
    elements), bit-exact against torch's own permute of the same tensor."""
    torch = torch_cuda
    import bench
    gen = torch.Generator(device="cuda").manual_seed(5)
    for expr, shape in bench.PERMUTES_4D:
        u = eir.unary_dims(expr, dict(zip("abcd", shape)))
        x = torch.rand(shape, device="cuda", generator=gen)
        y = torch.empty(x.numel(), device="cuda")
        plan = eir.PermutePlan(u["sizes"], u["strides_in"], u["strides_out"], dtype=eir.FP32, ktype=eir.COPY)
        plan.execute(x, y, stream=torch.cuda.current_stream())
        torch.cuda.synchronize()
        desc = plan.describe()
        plan.close()
        perm = ["abcd".index(ch) for ch in expr.split("->")[1]]
        assert torch.equal(y, x.permute(*perm).contiguous().view(-1)), (expr, shape, desc)


@pytest.mark.parametrize("pad", [0, 4])
def test_permute_padded_shared_unit_dim(torch_cuda, oracle, pad):
    """A shared unit-stride dim of 36 (b a d <- a b d) whose neighbours sit
    36 + pad elements apart in both tensors: packed, the row tiles span b and
    a; padded, no run extends past d and the vectorised copy moves it.  Gaps
    of the output keep their initial values."""
    torch = torch_cuda
    a, b, d = 5, 7, 36
    row = d + pad
    sizes = [b, a, d]                                   # output order
    s_in = [row, row * b, 1]
    s_out = [row * a, row, 1]
    n = row * a * b
    rng = np.random.default_rng(11 + pad)
    x = rng.uniform(-1, 1, n).astype(np.float32)
    o0 = rng.uniform(-1, 1, n).astype(np.float32)
    ref = o0.copy()
    oracle.permute(sizes, s_in, s_out, x, ref)
    plan = eir.PermutePlan(sizes, s_in, s_out, dtype=eir.FP32, ktype=eir.COPY)
    dx, do = _to_dev(torch, x), _to_dev(torch, o0)
    plan.execute(dx, do, stream=torch.cuda.current_stream())
    torch.cuda.synchronize()
    desc = plan.describe()
    plan.close()
    np.testing.assert_array_equal(do.cpu().numpy(), ref, err_msg=desc)
    assert ("rows" in desc) == (pad == 0), desc
