"""CPU tests of the etops-compatible API's configuration layer
(einsum_ir_amd.etops): validation rules, JSON round trip, file I/O and
optimize, as the reference states them (reference python/src/etops/__init__.py:
116-268 validation, 269-360 JSON, 436-514 optimize).  No GPU is needed: no plan
is created."""
import json

import pytest

from einsum_ir_amd import etops


def _gemm(**kw):
    # column-major GEMM C[m,n] = A[m,k] B[k,n] with m fastest: loops (m, n, k)
    base = dict(data_type=etops.float32, prim_first=etops.prim.zero, prim_main=etops.prim.gemm,
                prim_last=etops.prim.none, dim_types=(etops.dim.m, etops.dim.n, etops.dim.k),
                exec_types=(etops.exec.prim,) * 3, dim_sizes=(32, 16, 8),
                strides=(((1, 0, 32), (0, 8, 1), (1, 32, 0)),))
    base.update(kw)
    return etops.TensorOperationConfig(**base)


def test_enum_values_match_reference():
    # TensorOperation.h:39-80 numbering
    assert [e.value for e in (etops.exec.seq, etops.exec.prim, etops.exec.shared, etops.exec.sfc)] == [0, 1, 2, 3]
    assert [p.value for p in (etops.prim.none, etops.prim.zero, etops.prim.copy, etops.prim.relu,
                              etops.prim.gemm, etops.prim.brgemm)] == [0, 1, 2, 3, 4, 5]
    assert [d.value for d in (etops.dim.c, etops.dim.m, etops.dim.n, etops.dim.k)] == [0, 1, 2, 3]
    assert (etops.float32.value, etops.float64.value) == (0, 1)
    assert etops.ErrorType.invalid_optimization_config.value == 3
    assert etops.dtype is etops.DataType and etops.exec is etops.etype


def test_valid_configs():
    _gemm()
    _gemm(prim_main=etops.prim.brgemm, prim_last=etops.prim.relu)
    _gemm(backend="hip")
    etops.TensorOperationConfig(data_type=etops.float64, prim_first=etops.prim.none, prim_main=etops.prim.copy,
                                prim_last=etops.prim.none, dim_types=(etops.dim.c, etops.dim.c),
                                exec_types=(etops.exec.seq, etops.exec.seq), dim_sizes=(3, 4),
                                strides=(((4, 1), (1, 3)),))


@pytest.mark.parametrize("kw,rule", [
    (dict(backend="tpp"), "backend"),
    (dict(prim_main=etops.prim.relu), "prim_main"),
    (dict(prim_main=etops.prim.none), "prim_main"),
    (dict(exec_types=(etops.exec.prim,) * 2), "exec_types"),
    (dict(dim_sizes=(32, 16)), "dim_sizes"),
    (dict(dim_sizes=(32, 0, 8)), "dim_size_positive"),
    (dict(dim_sizes=(32, 16, -1)), "dim_size_positive"),
    (dict(strides=()), "stride_levels"),
    (dict(strides=(((1, 0, 32), (0, 8, 1)),)), "stride_tensors"),
    (dict(strides=(((1, 0, 32), (0, 8, 1), (1, 32, 0), (1, 1, 1)),)), "stride_tensors"),
    (dict(strides=(((1, 0), (0, 8, 1), (1, 32, 0)),)), "stride_dims"),
    (dict(prim_first=etops.prim.relu), "prim_first"),
    (dict(prim_first=etops.prim.copy), "prim_first"),
    (dict(prim_last=etops.prim.zero), "prim_last"),
    (dict(prim_last=etops.prim.gemm), "prim_last"),
])
def test_invalid_binary_configs(kw, rule):
    with pytest.raises(ValueError) as e:
        _gemm(**kw)
    assert e.value.rules == (rule,)


def test_binary_dims_and_levels_are_free():
    """Binary operations take any dim types, packing levels beyond level 0
    and every exec type."""
    _gemm(dim_types=(etops.dim.c, etops.dim.c, etops.dim.c))
    _gemm(strides=(((1, 0, 32), (0, 8, 1), (1, 32, 0)), ((0, 0, 0),)))
    _gemm(exec_types=(etops.exec.seq, etops.exec.shared, etops.exec.sfc))


def test_every_broken_rule_is_reported():
    with pytest.raises(ValueError) as e:
        _gemm(backend="cpu", dim_sizes=(0, 16), prim_last=etops.prim.copy)
    assert e.value.rules == ("backend", "dim_sizes", "dim_size_positive", "prim_last")
    # without a level 0 the stride shape rules that read it are not applied
    with pytest.raises(ValueError) as e:
        _gemm(strides=(), prim_first=etops.prim.relu)
    assert e.value.rules == ("stride_levels", "prim_first")
    # an unknown main primitive leaves nothing to check the kind-specific rules against
    with pytest.raises(ValueError) as e:
        _gemm(prim_main=etops.prim.relu, prim_first=etops.prim.relu, strides=(((1,),),))
    assert e.value.rules == ("prim_main",)


_COPY = dict(data_type=etops.float32, prim_first=etops.prim.none, prim_main=etops.prim.copy,
             prim_last=etops.prim.none, dim_types=(etops.dim.c, etops.dim.c),
             exec_types=(etops.exec.seq,) * 2, dim_sizes=(3, 4), strides=(((4, 1), (1, 3)),))


@pytest.mark.parametrize("kw,rule", [
    (dict(dim_types=(etops.dim.c, etops.dim.m)), "dim_types"),
    (dict(dim_types=(etops.dim.k, etops.dim.c)), "dim_types"),
    (dict(prim_first=etops.prim.zero), "prim_first"),
    (dict(prim_last=etops.prim.relu), "prim_last"),
    (dict(strides=(((4, 1), (1, 3), (1, 3)),)), "stride_tensors"),
    (dict(strides=(((4, 1), (1, 3, 9)),)), "stride_dims"),
])
def test_invalid_unary_configs(kw, rule):
    with pytest.raises(ValueError) as e:
        etops.TensorOperationConfig(**{**_COPY, **kw})
    assert e.value.rules == (rule,)


def test_unary_zero_is_accepted():
    etops.TensorOperationConfig(**{**_COPY, "prim_main": etops.prim.zero})


def test_json_round_trip(tmp_path):
    cfg = _gemm(prim_last=etops.prim.relu, backend="hip")
    s = cfg.to_json()
    data = json.loads(s)
    assert data["prim_last"] == "relu" and data["backend"] == "hip"
    assert data["dim_types"] == ["m", "n", "k"] and data["strides"] == [[[1, 0, 32], [0, 8, 1], [1, 32, 0]]]
    assert etops.TensorOperationConfig.from_json(s) == cfg
    path = tmp_path / "cfg.json"
    cfg.save(str(path))
    assert etops.TensorOperationConfig.load(str(path)) == cfg
    assert "backend" not in json.loads(_gemm().to_json())
    assert etops.TensorOperationConfig.from_json(_gemm().to_json()).backend is None


def test_json_rejects():
    with pytest.raises(ValueError) as e:
        etops.TensorOperationConfig.from_json('{"data_type": "float32"}')
    assert set(e.value.rules) == {"json_field"} and len(e.value.rules) == 7
    s = _gemm(prim_last=etops.prim.relu).to_json()
    with pytest.raises(ValueError) as e:
        etops.TensorOperationConfig.from_json(s.replace('"relu"', '"gelu"'))
    assert e.value.rules == ("json_value",)
    with pytest.raises(ValueError) as e:
        etops.TensorOperationConfig.from_json(s.replace('"k"', '"q"'))
    assert e.value.rules == ("json_value",)
    # a well-formed file whose content breaks a rule is rejected by the rule
    with pytest.raises(ValueError) as e:
        etops.TensorOperationConfig.from_json(s.replace('"relu"', '"zero"'))
    assert e.value.rules == ("prim_last",)


def _offsets(cfg):
    """The multiset of (offset in each tensor) tuples over every point of the
    config's iteration space: two configs with equal multisets multiply the
    same element pairs and add each product into the same output element."""
    import itertools
    sizes, strides = cfg.dim_sizes, cfg.strides[0]
    return sorted(tuple(sum(i * s for i, s in zip(idx, st)) for st in strides)
                  for idx in itertools.product(*map(range, sizes)))


def test_optimize_fuses_contiguous_loops():
    # out[b][c][m1][m2][n], A[b][c][m1][m2][k1][k2], B[b][c][n][k1][k2], plus
    # a size-1 loop x; b,c / m1,m2 / k1,k2 are contiguous in every tensor
    sizes = dict(b=2, c=3, m1=4, x=1, m2=5, n=6, k1=7, k2=8)
    d = etops.dim
    types = (d.c, d.c, d.m, d.n, d.m, d.n, d.k, d.k)
    a = dict(b=3360, c=1120, m1=280, x=0, m2=56, n=0, k1=8, k2=1)
    b = dict(b=1008, c=336, m1=0, x=0, m2=0, n=56, k1=8, k2=1)
    o = dict(b=360, c=120, m1=30, x=99, m2=6, n=1, k1=0, k2=0)
    names = list(sizes)
    cfg = _gemm(dim_types=types, exec_types=(etops.exec.seq,) * 8, dim_sizes=tuple(sizes.values()),
                strides=(tuple(tuple(t[n] for n in names) for t in (a, b, o)),))
    opt = etops.optimize(cfg)
    assert opt.dim_types == (d.c, d.m, d.n, d.k)
    assert opt.dim_sizes == (6, 20, 6, 56)
    assert opt.exec_types == (etops.exec.shared, etops.exec.prim, etops.exec.prim, etops.exec.prim)
    assert opt.strides == (((1120, 56, 0, 1), (336, 0, 56, 1), (120, 6, 1, 0)),)
    assert _offsets(opt) == _offsets(cfg)
    # the optimized config is valid and optimizes to itself
    assert etops.optimize(opt) == opt


def test_optimize_keeps_non_contiguous_loops():
    # A's m1 stride padded (300, not 64 * 4): m1 and m2 stay apart
    d = etops.dim
    cfg = _gemm(dim_types=(d.m, d.m, d.n, d.k), exec_types=(etops.exec.prim,) * 4, dim_sizes=(3, 4, 5, 7),
                strides=(((300, 64, 0, 1), (0, 0, 7, 1), (20, 5, 1, 0)),))
    opt = etops.optimize(cfg)
    assert opt.dim_sizes == (3, 4, 5, 7)
    assert _offsets(opt) == _offsets(cfg)
    # the same with A unpadded fuses m1, m2
    cfg = _gemm(dim_types=(d.m, d.m, d.n, d.k), exec_types=(etops.exec.prim,) * 4, dim_sizes=(3, 4, 5, 7),
                strides=(((28 * 4, 28, 0, 1), (0, 0, 7, 1), (20, 5, 1, 0)),))
    opt = etops.optimize(cfg)
    assert opt.dim_sizes == (12, 5, 7) and opt.strides[0][0] == (28, 0, 1)
    assert _offsets(opt) == _offsets(cfg)


def test_optimize_unary():
    # out[c1][c2][c3] = in[c3][c1][c2]: c1,c2 contiguous in both, c3 not
    d = etops.dim
    cfg = etops.TensorOperationConfig(data_type=etops.float32, prim_first=etops.prim.none,
                                      prim_main=etops.prim.copy, prim_last=etops.prim.none,
                                      dim_types=(d.c,) * 3, exec_types=(etops.exec.seq,) * 3, dim_sizes=(3, 4, 5),
                                      strides=(((4, 1, 12), (20, 5, 1)),))
    opt = etops.optimize(cfg)
    assert opt.dim_sizes == (12, 5) and opt.strides == (((1, 12), (5, 1)),)
    assert opt.exec_types == (etops.exec.prim,) * 2
    assert _offsets(opt) == _offsets(cfg)


def test_optimize():
    cfg = _gemm(exec_types=(etops.exec.seq, etops.exec.shared, etops.exec.sfc))
    opt = etops.optimize(cfg)
    assert opt.backend == "hip"
    # nothing to fuse: the loops come back as given, all inside the kernel
    assert opt.exec_types == (etops.exec.prim,) * 3
    assert opt.dim_sizes == cfg.dim_sizes and opt.dim_types == tuple(cfg.dim_types)
    assert opt.strides == (tuple(tuple(t) for t in cfg.strides[0]),)
    etops.optimize(cfg, {"target_m": 64, "packing_support": False})
    with pytest.raises(RuntimeError, match="invalid_optimization_config"):
        etops.optimize(cfg, {"not_a_key": 1})
    with pytest.raises(RuntimeError, match="invalid_optimization_config"):
        etops.optimize(cfg, {"target_m": "large"})
    defaults = etops.backend.hip.get_default_optimization_config()
    assert set(defaults) == {"target_m", "target_n", "target_k", "num_threads", "packed_gemm_support",
                             "br_gemm_support", "packing_support", "sfc_support", "l2_cache_size"}
