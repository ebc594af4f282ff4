"""GPU parity of the binary-contraction path (etir_hip_contraction_*).

Mirrors the reference's operator tests (reference
src/backend/BinaryContractionTpp.test.torch.cpp: matmul, bias COPY with
full/row/col/scalar broadcast, batched kmc,nkc->nmc, 7-D C/M/N/K, ZERO+RELU,
stride-1 C) and adds the BASELINE configs.  Checker: the CPU oracle (fp64
accumulation) on identical seeded inputs.  Bars: fp32 relative Frobenius
<= 1e-5; bf16 inputs (fp32 accumulate) <= 2e-3 against the exact result on
the same bf16-rounded inputs.
"""
import numpy as np
import pytest

import einsum_ir_amd as eir
from tests.helpers import TOL_FP32, TOL_BF16, TOL_FP64, parse_binary, tensor_numel, rel_frobenius, loops_for

pytestmark = pytest.mark.gpu


def _dev(torch, x):
    if x.dtype == np.uint16:
        return torch.from_numpy(x.view(np.int16)).cuda()
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def run_case(torch, oracle, expr, sizes, dtype=eir.FP32, first=eir.ZERO, last=eir.UNDEFINED_KTYPE,
             aux_outer=None, seed=0, dtype_out=eir.FP32, check=True):
    left, right, out = parse_binary(expr)
    loops = loops_for(expr, sizes, sizes_outer_aux=aux_outer)
    rng = np.random.default_rng(seed)
    npt = np.float64 if dtype == eir.FP64 else np.float32
    if dtype == eir.FP64:
        dtype_out = eir.FP64
    a = rng.uniform(-1, 1, tensor_numel(left, sizes)).astype(npt)
    b = rng.uniform(-1, 1, tensor_numel(right, sizes)).astype(npt)
    o0 = rng.uniform(-1, 1, tensor_numel(out, sizes)).astype(npt)
    needs_aux = first in (eir.COPY, eir.ADD) or last == eir.ADD
    x = rng.uniform(-1, 1, tensor_numel(out, aux_outer or sizes)).astype(npt) if needs_aux else None
    if dtype == eir.BF16:
        a, b = oracle.f32_to_bf16(a), oracle.f32_to_bf16(b)
    if dtype_out == eir.BF16:
        o0 = oracle.f32_to_bf16(o0)
        x = oracle.f32_to_bf16(x) if x is not None else None
    plan = eir.ContractionPlan(loops["dim_types"], loops["sizes"], loops["strides_left"],
                               loops["strides_right"], loops["strides_out"],
                               strides_out_aux=loops["strides_out_aux"],
                               dtype_left=dtype, dtype_right=dtype,
                               dtype_comp=eir.FP64 if dtype == eir.FP64 else eir.FP32,
                               dtype_out=dtype_out, ktype_first_touch=first, ktype_last_touch=last)
    da, db, do = _dev(torch, a), _dev(torch, b), _dev(torch, o0)
    dx = _dev(torch, x) if x is not None else None
    plan.execute(da, db, do, aux=dx, stream=torch.cuda.current_stream())
    torch.cuda.synchronize()
    got = do.cpu().numpy()
    desc = plan.describe()
    plan.close()
    if not check:
        return got, desc
    ref = o0.copy()
    oracle.contract(loops, a, b, ref, aux=x, dtype_left=dtype, dtype_right=dtype,
                    dtype_out=dtype_out, first_touch=first, last_touch=last)
    if dtype_out == eir.BF16:
        got = oracle.bf16_to_f32(got.view(np.uint16))
        ref = oracle.bf16_to_f32(ref)
    err = rel_frobenius(ref, got)
    tol = TOL_BF16 if (dtype == eir.BF16 or dtype_out == eir.BF16) else TOL_FP32
    if dtype == eir.FP64:
        tol = TOL_FP64
    assert err <= tol, f"{expr} {sizes}: rel. Frobenius error {err:.3e} > {tol:.0e} [{desc}]"
    return got, desc


def test_c1_abkl_cdkl_fp32(torch_cuda, oracle):
    """BASELINE config 1 at full size."""
    _, desc = run_case(torch_cuda, oracle, "abkl,cdkl->abcd", dict(a=32, b=16, c=32, d=16, k=32, l=16), seed=1)
    assert "vec_k" in desc


def test_c3_scaled_bf16(torch_cuda, oracle):
    """BASELINE config 3 layout with z and a/b reduced so the oracle stays fast."""
    _, desc = run_case(torch_cuda, oracle, "zakm,zbkn->zabmn",
                       dict(z=2, a=4, m=64, b=4, n=64, k=1024), dtype=eir.BF16, seed=3)
    assert "vec_mn" in desc


def test_c3_full_size_every_output(torch_cuda, oracle):
    """BASELINE config 3 at full size, every one of the 134M outputs checked.

    The output starts as NaN, so an element no tile writes fails.  Two fp64
    invariants over all outputs catch a tile, row or column written to the
    wrong place or with the wrong operands:
      sum_n out[z,a,b,m,n] = sum_k A[z,a,k,m] * (sum_n B[z,b,k,n])
      sum_m out[z,a,b,m,n] = sum_k (sum_m A[z,a,k,m]) * B[z,b,k,n]
    each compared element by element (deviation <= 1e-4 of the invariant's
    RMS; the fp32 accumulation error is ~1e-6 of it, one misplaced row ~1).
    4096 sampled outputs are also checked against fp64 dot products."""
    torch = torch_cuda
    sizes = dict(z=8, a=64, m=64, b=64, n=64, k=1024)
    loops = loops_for("zakm,zbkn->zabmn", sizes)
    rng = np.random.default_rng(33)
    a = oracle.f32_to_bf16(rng.uniform(-1, 1, 8 * 64 * 1024 * 64).astype(np.float32))
    b = oracle.f32_to_bf16(rng.uniform(-1, 1, 8 * 64 * 1024 * 64).astype(np.float32))
    plan = eir.ContractionPlan(loops["dim_types"], loops["sizes"], loops["strides_left"],
                               loops["strides_right"], loops["strides_out"], dtype_left=eir.BF16,
                               dtype_right=eir.BF16)
    assert "bf16_dma_256x256" in plan.describe()
    out = torch.full((8 * 64 * 64 * 64 * 64,), float("nan"), dtype=torch.float32, device="cuda")
    plan.execute(_dev(torch, a), _dev(torch, b), out, stream=torch.cuda.current_stream())
    torch.cuda.synchronize()
    plan.close()
    got = out.cpu().numpy().reshape(8, 64, 64, 64, 64)
    del out
    assert np.all(np.isfinite(got)), "unwritten or non-finite outputs"
    A = oracle.bf16_to_f32(a).reshape(8, 64, 1024, 64).astype(np.float64)
    B = oracle.bf16_to_f32(b).reshape(8, 64, 1024, 64).astype(np.float64)

    def check(inv_got, inv_ref, what):
        dev = np.abs(inv_got - inv_ref)
        scale = np.sqrt(np.mean(inv_ref ** 2))
        worst = np.unravel_index(np.argmax(dev), dev.shape)
        assert dev[worst] <= 1e-4 * scale, f"{what}: deviation {dev[worst]:.3e} at {worst} (RMS {scale:.3e})"

    # sum over n: [z,a,b,m]
    bs = B.sum(axis=3)                                        # [z,b,k]
    ref_n = np.einsum("zakm,zbk->zabm", A, bs, optimize=True)
    check(got.sum(axis=4, dtype=np.float64), ref_n, "sum over n")
    del ref_n, bs
    # sum over m: [z,a,b,n]
    as_ = A.sum(axis=3)                                       # [z,a,k]
    ref_m = np.einsum("zak,zbkn->zabn", as_, B, optimize=True)
    check(got.sum(axis=3, dtype=np.float64), ref_m, "sum over m")
    del ref_m, as_

    idx = [rng.integers(0, s, 4096) for s in (8, 64, 64, 64, 64)]
    z, ia, ib, im, inn = idx
    ref = np.einsum("sk,sk->s", A[z, ia, :, im], B[z, ib, :, inn])
    g = got[z, ia, ib, im, inn]
    assert rel_frobenius(ref, g) <= TOL_BF16


def test_mlp_layer_fp32(torch_cuda, oracle):
    """One layer of BASELINE config 4 (bi,ih->bh) at full size vs float64 matmul."""
    torch = torch_cuda
    sizes = dict(b=4096, i=2048, h=2048)
    rng = np.random.default_rng(4)
    x = rng.standard_normal(4096 * 2048).astype(np.float32)
    w = (rng.standard_normal(2048 * 2048) / np.sqrt(2048)).astype(np.float32)
    # the tree path swaps the inputs (fastest output dim is N): left=ih, right=bi
    loops = loops_for("ih,bi->bh", sizes)
    plan = eir.ContractionPlan(loops["dim_types"], loops["sizes"], loops["strides_left"],
                               loops["strides_right"], loops["strides_out"])
    out = torch.empty(4096 * 2048, dtype=torch.float32, device="cuda")
    plan.execute(_dev(torch, w), _dev(torch, x), out, stream=torch.cuda.current_stream())
    torch.cuda.synchronize()
    desc = plan.describe()
    plan.close()
    ref = x.astype(np.float64).reshape(4096, 2048) @ w.astype(np.float64).reshape(2048, 2048)
    err = rel_frobenius(ref, out.cpu().numpy())
    assert err <= TOL_FP32, f"{err} {desc}"


# reference operator-test shapes (BinaryContractionTpp.test.torch.cpp) + layout variety
SHAPES = [
    ("km,nk->nm", dict(k=37, m=65, n=33)),                     # matmul, ragged
    ("mk,kn->mn", dict(m=128, k=96, n=128)),
    ("ab,bc->ac", dict(a=5, b=3, c=7)),                        # tiny
    ("kmc,nkc->nmc", dict(k=9, m=17, c=6, n=11)),              # stride-1 C (packed GEMM case)
    ("cakm,cbkn->cabmn", dict(c=2, a=3, k=40, m=8, b=2, n=12)),
    ("abcde,fgchb->agdef", dict(a=3, b=4, c=5, d=2, e=7, f=3, g=2, h=4)),
    ("iabk,kjc->ijbca", dict(i=2, a=5, b=3, k=19, j=4, c=6)),  # 7-D C/M/N/K mixes
    ("bi,ih->bh", dict(b=130, i=70, h=66)),
    ("xay,yab->xab", dict(x=7, a=4, y=13, b=9)),
]


@pytest.mark.parametrize("expr,sizes", SHAPES)
@pytest.mark.parametrize("dtype", [eir.FP32, eir.BF16])
def test_layouts(torch_cuda, oracle, expr, sizes, dtype):
    run_case(torch_cuda, oracle, expr, sizes, dtype=dtype, seed=sum(map(ord, expr)))


@pytest.mark.parametrize("first,last", [(eir.COPY, eir.UNDEFINED_KTYPE), (eir.ADD, eir.UNDEFINED_KTYPE),
                                        (eir.UNDEFINED_KTYPE, eir.UNDEFINED_KTYPE), (eir.ZERO, eir.RELU),
                                        (eir.COPY, eir.RELU), (eir.ZERO, eir.ADD)])
@pytest.mark.parametrize("dtype", [eir.FP32, eir.BF16])
def test_touch_kernels(torch_cuda, oracle, first, last, dtype):
    run_case(torch_cuda, oracle, "km,nk->nm", dict(k=64, m=96, n=80), dtype=dtype, first=first, last=last)


@pytest.mark.parametrize("bcast", ["row", "col", "scalar"])
def test_copy_broadcast(torch_cuda, oracle, bcast):
    aux_outer = {"row": dict(m=1, n=48), "col": dict(m=40, n=1), "scalar": dict(m=1, n=1)}[bcast]
    aux_outer = dict(aux_outer, k=24)
    run_case(torch_cuda, oracle, "mk,kn->mn", dict(m=40, k=24, n=48), first=eir.COPY, aux_outer=aux_outer)


def test_bf16_output(torch_cuda, oracle):
    run_case(torch_cuda, oracle, "mk,nk->mn", dict(m=96, k=128, n=64), dtype=eir.BF16,
             dtype_out=eir.BF16, first=eir.ZERO)


def test_large_k_fp32(torch_cuda, oracle):
    run_case(torch_cuda, oracle, "mk,nk->mn", dict(m=64, k=8192, n=64))


def test_zero_k(torch_cuda, oracle):
    # K = 0: the first-touch result only (ZERO -> zeros, COPY -> aux)
    got, _ = run_case(torch_cuda, oracle, "mk,kn->mn", dict(m=8, k=0, n=8), check=False)
    assert not np.any(got)


def test_rejects_mixed_fp64(torch_cuda):
    loops = loops_for("mk,kn->mn", dict(m=4, k=4, n=4))
    with pytest.raises(eir.EinsumIrError) as e:
        eir.ContractionPlan(loops["dim_types"], loops["sizes"], loops["strides_left"],
                            loops["strides_right"], loops["strides_out"], dtype_left=eir.FP64,
                            dtype_right=eir.FP64, dtype_comp=eir.FP64, dtype_out=eir.FP32)
    assert e.value.code == eir.INVALID_DTYPE


def test_missing_aux_is_an_error(torch_cuda):
    torch = torch_cuda
    loops = loops_for("mk,kn->mn", dict(m=4, k=4, n=4))
    plan = eir.ContractionPlan(loops["dim_types"], loops["sizes"], loops["strides_left"],
                               loops["strides_right"], loops["strides_out"], ktype_first_touch=eir.COPY)
    t = torch.zeros(16, device="cuda")
    with pytest.raises(eir.EinsumIrError) as e:
        plan.execute(t, t, t)
    assert e.value.code == eir.NO_DATA_PTR_PROVIDED
    plan.close()


# every tile configuration on layouts that exercise all load modes, ragged edges
# and the affine / table K paths (ETIR_TILE overrides the planner's tile choice)
TILES_F32 = [0, 1]
TILES_BF16 = [2, 6, 3, 4]
TILE_SHAPES = [
    ("zakm,zbkn->zabmn", dict(z=2, a=3, m=64, b=2, n=64, k=96)),   # vec_mn x vec_mn, affine K
    ("mk,nk->mn", dict(m=300, k=72, n=260)),                       # vec_k x vec_k, ragged
    ("km,nk->nm", dict(k=40, m=136, n=200)),                       # vec_mn x vec_k
    ("akbl,cldk->abcd", dict(a=5, b=7, c=6, d=9, k=12, l=8)),      # table K, scalar loads
]


@pytest.mark.parametrize("tile", TILES_F32 + TILES_BF16)
@pytest.mark.parametrize("expr,sizes", TILE_SHAPES)
def test_every_tile(torch_cuda, oracle, monkeypatch, tile, expr, sizes):
    monkeypatch.setenv("ETIR_TILE", str(tile))
    dtype = eir.FP32 if tile in TILES_F32 else eir.BF16
    _, desc = run_case(torch_cuda, oracle, expr, sizes, dtype=dtype, seed=tile * 7 + len(expr))
    names = {0: "f32_128x128", 1: "f32_64x64", 2: "bf16_256x256", 6: "bf16_256x128",
             3: "bf16_128x128", 4: "bf16_64x64"}
    assert names[tile] in desc


@pytest.mark.parametrize("tile", TILES_F32 + TILES_BF16)
@pytest.mark.parametrize("k", [5, 40, 100])
def test_every_tile_k_tail(torch_cuda, oracle, monkeypatch, tile, k):
    """The last k step runs only its fragment steps that hold valid k (5, 8 or
    4 of 32; 5, 40 or 36 of 64): results as with the full step."""
    monkeypatch.setenv("ETIR_TILE", str(tile))
    dtype = eir.FP32 if tile in TILES_F32 else eir.BF16
    run_case(torch_cuda, oracle, "km,kn->mn", dict(k=k, m=136, n=264), dtype=dtype, seed=tile + k)


# a short M side (24) against a long N: every tile is an edge tile of the
# direct-store epilogue; K = 36 and 40 leave most of the last k step padding
SHORT_M_SHAPES = [
    ("ebadf,cf->abcde", dict(a=8, b=8, c=24, d=16, e=64, f=36)),     # vec_k x vec_k, K = 36
    ("efbad,cf->abcde", dict(a=8, b=8, c=24, d=16, e=64, f=36)),     # scalar N-side loads
    ("dbea,ec->abcd", dict(a=64, b=33, c=24, d=31, e=40)),           # ragged N
    ("mk,kn->mn", dict(m=32, k=40, n=70000)),                        # one full row of tiles, ragged N
]


@pytest.mark.parametrize("expr,sizes", SHORT_M_SHAPES)
@pytest.mark.parametrize("first,last", [(eir.ZERO, eir.UNDEFINED_KTYPE), (eir.ZERO, eir.RELU),
                                        (eir.ADD, eir.UNDEFINED_KTYPE)])
def test_short_m(torch_cuda, oracle, expr, sizes, first, last):
    run_case(torch_cuda, oracle, expr, sizes, first=first, last=last, seed=len(expr) + first)


@pytest.mark.parametrize("nt", ["0", "1"])
@pytest.mark.parametrize("tile", [0, 1])
@pytest.mark.parametrize("expr,sizes", [
    ("mk,kn->mn", dict(m=100, k=40, n=300)),                         # unit-stride columns, ragged
    ("eax,ebcdx->abcdx", dict(e=12, a=9, b=5, c=6, d=7, x=8)),       # columns 8 apart (C innermost)
    ("dega,gfbc->abcdef", dict(a=3, b=4, c=5, d=6, e=7, f=9, g=10)), # columns in runs of 9
])
def test_edge_tile_direct_stores(torch_cuda, oracle, monkeypatch, nt, tile, expr, sizes):
    """Edge tiles with a ZERO first touch store straight from the
    accumulators with the rows and columns past M and N masked off; the
    stores are non-temporal or not (forced either way here) -- same results."""
    monkeypatch.setenv("ETIR_OUT_NT", nt)
    monkeypatch.setenv("ETIR_TILE", str(tile))
    for last in (eir.UNDEFINED_KTYPE, eir.RELU):
        run_case(torch_cuda, oracle, expr, sizes, last=last, seed=tile + int(nt))


@pytest.mark.parametrize("expr,sizes", [
    ("efbadx,cfx->abcdex", dict(e=6, f=8, b=5, a=4, d=6, c=7, x=16)),
    ("eax,ebcdx->abcdx", dict(e=12, a=9, b=5, c=6, d=7, x=8)),
])
@pytest.mark.parametrize("dtype", [eir.FP32, eir.BF16, eir.FP64])
def test_batch_innermost_output(torch_cuda, oracle, expr, sizes, dtype):
    """A C dim innermost in the output (TCCG's x-batch cases): workgroups walk
    C fastest; results as for any other order."""
    _, desc = run_case(torch_cuda, oracle, expr, sizes, dtype=dtype, seed=5)
    assert "c_inner" in desc, desc
