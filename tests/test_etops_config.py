"""CPU tests of the etops-compatible API's configuration layer
(einsum_ir_amd.etops): validation rules, JSON round trip, file I/O and
optimize, as the reference states them (reference python/src/etops/__init__.py:
116-268 validation, 269-360 JSON, 436-514 optimize).  No GPU is needed: no plan
is created."""
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


@pytest.mark.parametrize("kw,msg", [
    (dict(backend="tpp"), "Unsupported backend"),
    (dict(prim_main=etops.prim.relu), "Invalid prim_main"),
    (dict(exec_types=(etops.exec.prim,) * 2), "exec_types length"),
    (dict(dim_sizes=(32, 16)), "dim_sizes length"),
    (dict(dim_sizes=(32, 0, 8)), "must be positive"),
    (dict(strides=()), "at least one level"),
    (dict(strides=(((1, 0, 32), (0, 8, 1)),)), "must have 3 tensors"),
    (dict(strides=(((1, 0), (0, 8, 1), (1, 32, 0)),)), "length"),
    (dict(prim_first=etops.prim.relu), "prim_first must be"),
    (dict(prim_last=etops.prim.zero), "prim_last must be"),
])
def test_invalid_binary_configs(kw, msg):
    with pytest.raises(ValueError, match=msg):
        _gemm(**kw)


def test_invalid_unary_configs():
    base = dict(data_type=etops.float32, prim_first=etops.prim.none, prim_main=etops.prim.copy,
                prim_last=etops.prim.none, dim_types=(etops.dim.c, etops.dim.c),
                exec_types=(etops.exec.seq,) * 2, dim_sizes=(3, 4), strides=(((4, 1), (1, 3)),))
    with pytest.raises(ValueError, match="all dim_types must be"):
        etops.TensorOperationConfig(**{**base, "dim_types": (etops.dim.c, etops.dim.m)})
    with pytest.raises(ValueError, match="prim_first must be etops.prim.none"):
        etops.TensorOperationConfig(**{**base, "prim_first": etops.prim.zero})
    with pytest.raises(ValueError, match="must have 2 tensors"):
        etops.TensorOperationConfig(**{**base, "strides": (((4, 1), (1, 3), (1, 3)),)})


def test_json_round_trip(tmp_path):
    cfg = _gemm(prim_last=etops.prim.relu, backend="hip")
    s = cfg.to_json()
    assert '"prim_last": "relu"' in s and '"backend": "hip"' in s
    assert etops.TensorOperationConfig.from_json(s) == cfg
    path = tmp_path / "cfg.json"
    cfg.save(str(path))
    assert etops.TensorOperationConfig.load(str(path)) == cfg
    assert "backend" not in _gemm().to_json()
    with pytest.raises(ValueError, match="Missing required fields"):
        etops.TensorOperationConfig.from_json('{"data_type": "float32"}')
    with pytest.raises(ValueError, match="Invalid PrimType value"):
        etops.TensorOperationConfig.from_json(s.replace('"relu"', '"gelu"'))


def test_optimize():
    cfg = _gemm(exec_types=(etops.exec.seq, etops.exec.shared, etops.exec.sfc))
    opt = etops.optimize(cfg)
    assert opt.backend == "hip"
    assert opt.exec_types == (etops.exec.prim,) * 3
    assert opt.dim_sizes == cfg.dim_sizes and opt.dim_types == tuple(cfg.dim_types)
    assert opt.strides == (tuple(tuple(t) for t in cfg.strides[0]),)
    etops.optimize(cfg, {"target_m": 64, "packing_support": False})
    with pytest.raises(RuntimeError, match="invalid_optimization_config"):
        etops.optimize(cfg, {"not_a_key": 1})
    defaults = etops.backend.hip.get_default_optimization_config()
    assert set(defaults) == {"target_m", "target_n", "target_k", "num_threads", "packed_gemm_support",
                             "br_gemm_support", "packing_support", "sfc_support", "l2_cache_size"}
