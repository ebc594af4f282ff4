"""etops-compatible tensor operations on the HIP backend.

Mirrors the reference's Python module ``etops`` (reference
python/src/etops/__init__.py:1-532, python/src/bindings.cpp:10-334,
python/src/TensorOperation.{h,cpp}): the same enums and names,
``TensorOperationConfig`` with the same fields, validation, JSON form and
file I/O, ``TensorOperation.setup/execute``, ``optimize`` and
``backend.<name>.get_default_optimization_config``.  The backend is ``"hip"``
(``None`` selects it); the loop IR a config describes goes unchanged to the
C ABI of libeinsum_ir_hip.so (``etir_hip_contraction_create`` /
``etir_hip_permute_create``), which plans and runs it on the GPU.

Tensors: ``execute`` takes device arrays -- torch tensors on the GPU, objects
with ``__cuda_array_interface__`` or ``__dlpack__``, or raw device pointers
(int) -- and, like the reference, host numpy arrays, which are staged through
device buffers (copy in, run, copy back; a convenience, not a fast path).
``execute`` is synchronous like the reference's; ``execute_async`` enqueues on
a stream and returns.

Differences from the tpp backend, by design:
  * exec_types are validated and kept but do not steer execution: every loop
    of the operation is run by one kernel grid (the planner fuses loops and
    picks tiles itself);
  * level-1 (packing) strides are accepted and ignored: the kernels stage
    tiles through LDS instead of packing buffers;
  * ``optimize`` returns the loops as the GPU planner runs them (size-1 loops
    dropped, contiguous loops of one type fused; exec type ``shared`` for a
    contraction's C loops, which form the grid, ``prim`` otherwise) and no
    packing level; tpp's optimisation keys are accepted (and have no effect),
    unknown keys are rejected as in the reference;
  * DataType has the additive member ``bfloat16`` (bf16 tensors, fp32
    accumulation).
"""
import ctypes
import dataclasses
import enum
import json
from dataclasses import dataclass
from typing import Dict, Optional, Sequence, Union

from . import _lib
from ._lib import check, hip_lib


class ErrorType(enum.IntEnum):
    """TensorOperation::error_t (reference python/src/TensorOperation.h:74-80)."""
    success = 0
    compilation_failed = 1
    invalid_stride_shape = 2
    invalid_optimization_config = 3


class DataType(enum.IntEnum):
    """TensorOperation::dtype_t (:68-72); bfloat16 is additive."""
    float32 = 0
    float64 = 1
    bfloat16 = 2


class PrimType(enum.IntEnum):
    """TensorOperation::prim_t (:47-56)."""
    none = 0
    zero = 1
    copy = 2
    relu = 3
    gemm = 4
    brgemm = 5


class ExecType(enum.IntEnum):
    """TensorOperation::exec_t (:39-45)."""
    seq = 0
    prim = 1
    shared = 2
    sfc = 3


class DimType(enum.IntEnum):
    """TensorOperation::dim_t (:58-65)."""
    c = 0
    m = 1
    n = 2
    k = 3


dtype = DataType
float32 = DataType.float32
float64 = DataType.float64
bfloat16 = DataType.bfloat16


def _namespace(name: str, members: type, doc: str) -> type:
    """A plain class whose attributes are the members of an enum, so that
    ``etops.prim.gemm`` is ``PrimType.gemm``."""
    attrs = {m.name: m for m in members}
    return type(name, (), {**attrs, "__doc__": doc, "__all__": list(attrs)})


prim = _namespace("prim", PrimType, "Primitives of a tensor operation (first touch, main, last touch).")
etype = _namespace("etype", ExecType, "How a loop of a tensor operation is executed.")
exec = etype  # noqa: A001  (exported under both names, like the reference module)
dim = _namespace("dim", DimType, "The role of a dimension: batch c, rows m, columns n, reduction k.")

BACKENDS = ("hip",)
# the tpp backend's optimisation keys (reference bindings.cpp:174-178)
_OPT_KEYS = ("target_m", "target_n", "target_k", "num_threads", "packed_gemm_support",
             "br_gemm_support", "packing_support", "sfc_support", "l2_cache_size")


# ---------------------------------------------------------------------------
# configuration rules
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class _OpKind:
    """One kind of operation, selected by its main primitive, and what it
    allows around it (the accept/reject rules of reference etops/__init__.py:
    170-253 and TensorOperation.cpp:220-289, restated as data)."""
    name: str
    mains: frozenset
    tensors: tuple             # level-0 stride lists, in order
    firsts: frozenset          # allowed first-touch primitives
    lasts: frozenset           # allowed last-touch primitives
    dims: Optional[frozenset]  # allowed dimension types, None: any


_OP_KINDS = (
    _OpKind("binary", frozenset({PrimType.gemm, PrimType.brgemm}), ("in0", "in1", "out"),
            frozenset({PrimType.none, PrimType.zero}), frozenset({PrimType.none, PrimType.relu}), None),
    _OpKind("unary", frozenset({PrimType.copy, PrimType.zero}), ("in", "out"),
            frozenset({PrimType.none}), frozenset({PrimType.none}), frozenset({DimType.c})),
)


def _kind_of(prim_main) -> Optional[_OpKind]:
    return next((k for k in _OP_KINDS if prim_main in k.mains), None)


class ConfigError(ValueError):
    """A rejected configuration.  ``rules`` names every rule it breaks, in
    the order of the rule table; ``str()`` lists them with details."""

    def __init__(self, problems):
        self.rules = tuple(rule for rule, _ in problems)
        self.problems = tuple(problems)
        super().__init__("; ".join(f"[{rule}] {text}" for rule, text in problems))


def _bad_entries(values, ok):
    return [f"{i}: {v!r}" for i, v in enumerate(values) if not ok(v)]


def _stride_dims(cfg, kind):
    off = [f"{name} has {len(st)}" for name, st in zip(kind.tensors, cfg.strides[0])
           if len(st) != len(cfg.dim_types)]
    return f"{len(cfg.dim_types)} dims, but " + ", ".join(off) if off else None


# (rule, check).  A check gets the config and its operation kind and returns
# None when the rule holds, else a description.  Rules whose inputs an earlier
# rule found malformed are skipped (see _problems).
_RULES = (
    ("backend", lambda c, k: None if c.backend is None or c.backend in BACKENDS
        else f"backend {c.backend!r} is not one of {BACKENDS} (or None)"),
    ("prim_main", lambda c, k: None if k is not None
        else f"{c.prim_main!r} is no main primitive; binary: gemm, brgemm; unary: copy, zero"),
    ("exec_types", lambda c, k: None if len(c.exec_types) == len(c.dim_types)
        else f"{len(c.exec_types)} exec types for {len(c.dim_types)} dims"),
    ("dim_sizes", lambda c, k: None if len(c.dim_sizes) == len(c.dim_types)
        else f"{len(c.dim_sizes)} sizes for {len(c.dim_types)} dims"),
    ("dim_size_positive", lambda c, k: ", ".join(_bad_entries(c.dim_sizes, lambda s: s > 0)) or None),
    ("stride_levels", lambda c, k: None if len(c.strides) > 0 else "no level-0 strides"),
    ("stride_tensors", lambda c, k: None if len(c.strides[0]) == len(k.tensors)
        else f"level 0 holds {len(c.strides[0])} stride lists, a {k.name} operation takes "
             f"{len(k.tensors)} ({', '.join(k.tensors)})"),
    ("stride_dims", lambda c, k: _stride_dims(c, k)),
    ("dim_types", lambda c, k: None if k.dims is None else
        ", ".join(_bad_entries(c.dim_types, lambda d: d in k.dims)) or None),
    ("prim_first", lambda c, k: None if c.prim_first in k.firsts
        else f"{c.prim_first!r} cannot open a {k.name} operation"),
    ("prim_last", lambda c, k: None if c.prim_last in k.lasts
        else f"{c.prim_last!r} cannot close a {k.name} operation"),
)
# rules that need the operation kind, and the rule each further depends on
_NEEDS = {"stride_tensors": ("prim_main", "stride_levels"), "stride_dims": ("prim_main", "stride_levels"),
          "dim_types": ("prim_main",), "prim_first": ("prim_main",), "prim_last": ("prim_main",)}


def _problems(cfg) -> list:
    kind = _kind_of(cfg.prim_main)
    failed, found = set(), []
    for rule, check in _RULES:
        if any(dep in failed for dep in _NEEDS.get(rule, ())):
            continue
        text = check(cfg, kind)
        if text is not None:
            failed.add(rule)
            found.append((rule, text))
    return found


# ---------------------------------------------------------------------------
# JSON form: one codec per field (the keys and value spellings are the
# reference's file format, etops/__init__.py:269-360; "backend" is optional)
# ---------------------------------------------------------------------------
def _enum_codec(members):
    def decode(name):
        if name not in members.__members__:
            raise ConfigError([("json_value", f"{name!r} is not a {members.__name__} name")])
        return members[name]
    return (lambda v: v.name), decode


def _enum_list_codec(members):
    enc, dec = _enum_codec(members)
    return (lambda vs: [enc(v) for v in vs]), (lambda names: tuple(dec(n) for n in names))


_JSON_FIELDS = {
    "data_type": _enum_codec(DataType),
    "prim_first": _enum_codec(PrimType),
    "prim_main": _enum_codec(PrimType),
    "prim_last": _enum_codec(PrimType),
    "dim_types": _enum_list_codec(DimType),
    "exec_types": _enum_list_codec(ExecType),
    "dim_sizes": (list, tuple),
    "strides": (lambda s: [[list(t) for t in lvl] for lvl in s],
                lambda s: tuple(tuple(tuple(t) for t in lvl) for lvl in s)),
}


@dataclass(frozen=True)
class TensorOperationConfig:
    """Everything that defines one tensor operation (reference
    etops/__init__.py:116-268): data type, the three primitives, one entry per
    loop in dim_types / exec_types / dim_sizes, and strides indexed
    [level][tensor][loop].  Level 0 holds the tensors' own strides (binary:
    in0, in1, out; unary: in, out); further levels are packing strides, kept
    but not used by the GPU kernels.  A config that breaks a rule raises
    ConfigError (a ValueError) on construction."""
    data_type: DataType
    prim_first: PrimType
    prim_main: PrimType
    prim_last: PrimType
    dim_types: Sequence[DimType]
    exec_types: Sequence[ExecType]
    dim_sizes: Sequence[int]
    strides: Sequence[Sequence[Sequence[int]]]
    backend: Optional[str] = None

    def __post_init__(self):
        problems = _problems(self)
        if problems:
            raise ConfigError(problems)

    def apply(self, op: "TensorOperation") -> None:
        err = op.setup(self.backend if self.backend is not None else "hip", self.data_type, self.prim_first,
                       self.prim_main, self.prim_last, tuple(self.dim_types), tuple(self.exec_types),
                       tuple(self.dim_sizes),
                       tuple(tuple(tuple(t) for t in level) for level in self.strides))
        if err != ErrorType.success:
            raise RuntimeError(f"TensorOperation.setup returned {ErrorType(err).name}")

    def to_json(self, indent: Optional[int] = None) -> str:
        data = {key: encode(getattr(self, key)) for key, (encode, _) in _JSON_FIELDS.items()}
        if self.backend is not None:
            data["backend"] = self.backend
        return json.dumps(data, indent=indent)

    @classmethod
    def from_json(cls, json_str: str) -> "TensorOperationConfig":
        data = json.loads(json_str)
        absent = [key for key in _JSON_FIELDS if key not in data]
        if absent:
            raise ConfigError([("json_field", f"no {key!r}") for key in absent])
        fields = {key: decode(data[key]) for key, (_, decode) in _JSON_FIELDS.items()}
        return cls(backend=data.get("backend"), **fields)

    def save(self, path: str, indent: Optional[int] = 2) -> None:
        with open(path, "w") as f:
            f.write(self.to_json(indent=indent))

    @classmethod
    def load(cls, path: str) -> "TensorOperationConfig":
        with open(path) as f:
            return cls.from_json(f.read())

# ---------------------------------------------------------------------------
# tensors: device arrays, raw pointers, host numpy arrays (staged)
# ---------------------------------------------------------------------------
_NP_DTYPE = {DataType.float32: "float32", DataType.float64: "float64", DataType.bfloat16: None}


def _device_pointer(x):
    """Device address of a device array, or None when x is a host array."""
    if x is None:
        return 0
    if isinstance(x, int):
        return x
    try:
        import torch
        if isinstance(x, torch.Tensor):
            if not x.is_cuda:
                raise TypeError("etops (hip): torch tensors must live on the GPU")
            return x.data_ptr()
    except ImportError:
        pass
    iface = getattr(x, "__cuda_array_interface__", None)
    if iface is not None:
        return int(iface["data"][0])
    if hasattr(x, "__dlpack__") and hasattr(x, "__dlpack_device__"):
        dev_type, _ = x.__dlpack_device__()
        if dev_type in (2, 10):          # kDLCUDA, kDLROCM
            import torch
            return torch.from_dlpack(x).data_ptr()
    return None


class _Staged:
    """A host numpy array copied into a device buffer for one execute."""

    def __init__(self, array, np_dtype, writable):
        import numpy as np
        if writable:
            if not (isinstance(array, np.ndarray) and array.dtype == np_dtype and array.flags.c_contiguous
                    and array.flags.writeable):
                raise TypeError(f"etops (hip): the output must be a writable C-contiguous {np_dtype} array")
            self.host = array
        else:
            self.host = np.ascontiguousarray(array, dtype=np_dtype)
        self.nbytes = self.host.nbytes
        self.dev = ctypes.c_void_p()
        check(hip_lib().etir_hip_malloc(ctypes.byref(self.dev), self.nbytes))
        check(hip_lib().etir_hip_memcpy_h2d(self.dev, self.host.ctypes.data, self.nbytes))

    def copy_back(self):
        check(hip_lib().etir_hip_memcpy_d2h(self.host.ctypes.data, self.dev, self.nbytes))

    def free(self):
        if self.dev:
            hip_lib().etir_hip_free(self.dev)
            self.dev = ctypes.c_void_p()


# ---------------------------------------------------------------------------
# TensorOperation
# ---------------------------------------------------------------------------
_KT_FIRST = {PrimType.none: _lib.UNDEFINED_KTYPE, PrimType.zero: _lib.ZERO}
_KT_LAST = {PrimType.none: _lib.UNDEFINED_KTYPE, PrimType.relu: _lib.RELU}
_DT = {DataType.float32: (_lib.FP32, _lib.FP32, _lib.FP32, _lib.FP32),
       DataType.float64: (_lib.FP64, _lib.FP64, _lib.FP64, _lib.FP64),
       DataType.bfloat16: (_lib.BF16, _lib.BF16, _lib.FP32, _lib.BF16)}


class TensorOperation:
    """One unary or binary tensor operation compiled for the GPU
    (reference python/src/TensorOperation.cpp:220-479)."""

    def __init__(self, config: Union[TensorOperationConfig, None] = None):
        self._plan = None
        self._kind = None
        self._dtype = None
        if config is not None:
            config.apply(self)

    def close(self):
        if self._plan is not None:
            self._plan.close()
            self._plan = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def setup(self, backend, dtype, prim_first, prim_main, prim_last, dim_types, exec_types, dim_sizes,
              strides) -> ErrorType:
        """TensorOperation::setup (reference TensorOperation.cpp:220-289)."""
        self.close()
        if backend is not None and backend not in BACKENDS:
            return ErrorType.compilation_failed
        op_kind = _kind_of(PrimType(prim_main))
        if op_kind is None:
            return ErrorType.compilation_failed
        kind = op_kind.name
        n = len(dim_sizes)
        if len(strides) == 0 or len(strides[0]) != len(op_kind.tensors):
            return ErrorType.invalid_stride_shape
        if any(len(t) != n for t in strides[0]):
            return ErrorType.invalid_stride_shape
        if len(dim_types) != n or len(exec_types) != n:
            return ErrorType.compilation_failed
        dtype = DataType(dtype)
        try:
            if kind == "binary":
                if PrimType(prim_first) not in _KT_FIRST or PrimType(prim_last) not in _KT_LAST:
                    return ErrorType.compilation_failed
                dl, dr, dc, do = _DT[dtype]
                from . import ContractionPlan
                self._plan = ContractionPlan([int(DimType(d)) for d in dim_types], list(dim_sizes),
                                             list(strides[0][0]), list(strides[0][1]), list(strides[0][2]),
                                             dtype_left=dl, dtype_right=dr, dtype_comp=dc, dtype_out=do,
                                             ktype_first_touch=_KT_FIRST[PrimType(prim_first)],
                                             ktype_main=_lib.MADD,
                                             ktype_last_touch=_KT_LAST[PrimType(prim_last)])
            else:
                if PrimType(prim_first) != PrimType.none or PrimType(prim_last) != PrimType.none:
                    return ErrorType.compilation_failed
                # dims in output order (descending output stride), input strides alongside
                order = sorted(range(n), key=lambda i: -strides[0][1][i])
                from . import PermutePlan
                kt = _lib.COPY if PrimType(prim_main) == PrimType.copy else _lib.ZERO
                self._plan = PermutePlan([dim_sizes[i] for i in order], [strides[0][0][i] for i in order],
                                         [strides[0][1][i] for i in order], dtype=_DT[dtype][0], ktype=kt)
        except _lib.EinsumIrError:
            self._plan = None
            return ErrorType.compilation_failed
        self._kind = kind
        self._dtype = dtype
        self._extent = self._extents(dim_sizes, strides[0])
        return ErrorType.success

    @staticmethod
    def _extents(sizes, level0):
        """Elements spanned by each tensor (largest offset + 1)."""
        return [1 + sum((s - 1) * abs(st) for s, st in zip(sizes, t)) for t in level0]

    def describe(self) -> str:
        """The GPU plan's kernel choice (tile, fused loops, load modes)."""
        return self._plan.describe() if self._plan is not None else ""

    def execute_async(self, in0, in1, out, stream=None) -> None:
        """Enqueues the operation on `stream` (device arrays / pointers only)."""
        if self._plan is None:
            raise RuntimeError("einsum_ir TensorOperation: execute before a successful setup")
        ptrs = [_device_pointer(x) for x in (in0, in1, out)]
        if any(p is None for p in ptrs):
            raise TypeError("etops (hip): execute_async takes device arrays or device pointers")
        self._launch(*ptrs, stream)

    def _launch(self, p0, p1, pout, stream):
        if self._kind == "binary":
            self._plan.execute(p0, p1, pout, stream=stream)
        else:
            self._plan.execute(p0, pout, stream=stream)

    def execute(self, in0, in1=None, out=None) -> None:
        """TensorOperation::execute (reference TensorOperation.cpp:459-468): runs
        the operation and waits for it.  Device arrays run in place; host
        numpy arrays are staged through device buffers."""
        if out is None:
            raise TypeError("etops: execute needs an output tensor")
        if self._plan is None:
            raise RuntimeError("einsum_ir TensorOperation: execute before a successful setup")
        args = [in0, in1 if self._kind == "binary" else None, out]
        ptrs = [_device_pointer(x) for x in args]
        staged = []
        try:
            np_dtype = _NP_DTYPE[self._dtype]
            extents = self._extent if self._kind == "binary" else [self._extent[0], 0, self._extent[1]]
            for i, (x, p) in enumerate(zip(args, ptrs)):
                if p is not None:
                    continue
                if np_dtype is None:
                    raise TypeError("etops (hip): bfloat16 operations take device arrays only")
                st = _Staged(x, np_dtype, writable=(i == 2))
                if st.host.size < extents[i]:
                    raise ValueError(f"etops: tensor {i} holds {st.host.size} elements, the strides "
                                     f"address {extents[i]}")
                staged.append((i, st))
                ptrs[i] = st.dev.value
            self._launch(ptrs[0], ptrs[1], ptrs[2], None)
            check(hip_lib().etir_hip_synchronize(None))
            for i, st in staged:
                if i == 2:
                    st.copy_back()
        finally:
            for _, st in staged:
                st.free()

    @staticmethod
    def get_default_optimization_config(backend: str = "hip") -> Dict[str, Union[int, bool]]:
        if backend not in BACKENDS:
            return {}
        # tpp's keys with the GPU kernels' own figures: the largest tile and
        # K step, all threads of the device (0 = auto), no packing/SFC/BRGEMM
        # distinction (the planner decides per plan), the L2 of one XCD
        return {"target_m": 256, "target_n": 256, "target_k": 32, "num_threads": 0,
                "packed_gemm_support": False, "br_gemm_support": True, "packing_support": False,
                "sfc_support": False, "l2_cache_size": 4 * 1024 * 1024}


class _HIPBackend:
    """HIP (MI355X, gfx950) backend for tensor operations."""
    name: str = "hip"

    @staticmethod
    def get_default_optimization_config() -> Dict[str, Union[int, bool]]:
        return TensorOperation.get_default_optimization_config("hip")


class backend:
    """Namespace for available backends."""
    hip = _HIPBackend()


def optimize(config: TensorOperationConfig,
             optimization_config: Optional[Dict[str, Union[int, bool]]] = None) -> TensorOperationConfig:
    """Optimizes a configuration (reference etops/__init__.py:436-514,
    TensorOperation.cpp:486-604).  On the HIP backend the result is the loop
    IR the GPU planner runs: size-1 loops dropped, loops of one type that are
    contiguous in every tensor fused, exec type ``shared`` for the C loops of
    a contraction (the kernel grid) and ``prim`` for the loops inside the
    kernel (M, N, K; every loop of a permutation).  Tiles are chosen when the
    operation is set up.  Keys other than the tpp backend's raise like the
    reference's; their values have no effect."""
    actual = config.backend or "hip"
    if actual not in BACKENDS:
        raise ValueError(f"optimize: no backend {actual!r} here (only {BACKENDS})")
    options = backend.hip.get_default_optimization_config() if optimization_config is None else optimization_config
    rejected = [key for key, value in options.items() if key not in _OPT_KEYS or not isinstance(value, (int, bool))]
    if rejected:
        raise RuntimeError(f"optimize returned {ErrorType.invalid_optimization_config.name}: "
                           f"unknown key or non-integer value for {rejected}")
    dim_types, dim_sizes, strides = _fuse_loops(config.dim_types, config.dim_sizes, config.strides[0])
    binary = config.prim_main in (PrimType.gemm, PrimType.brgemm)
    exec_types = tuple(ExecType.shared if binary and t == DimType.c else ExecType.prim for t in dim_types)
    return dataclasses.replace(config, backend=actual, dim_types=dim_types, dim_sizes=dim_sizes,
                               exec_types=exec_types, strides=(strides,))


def _fuse_loops(dim_types, dim_sizes, strides):
    """The loops as the GPU planner runs them: loops of size 1 dropped (one is
    kept if nothing else is left), then any two loops of one type where the
    outer one's stride equals the inner one's stride times its size in every
    tensor merged into one loop of the product size, until none is left to
    merge (the fusion step of reference ContractionOptimizer.cpp:76-111, for a
    kernel that takes whole loop types at once, so no loop is split or
    reordered).  Returns (dim_types, dim_sizes, strides per tensor)."""
    loops = [[DimType(t), int(s), [int(st[i]) for st in strides]]
             for i, (t, s) in enumerate(zip(dim_types, dim_sizes)) if int(s) != 1]
    if not loops:
        loops = [[DimType(dim_types[0]), int(dim_sizes[0]), [int(st[0]) for st in strides]]] if dim_sizes else []
    merged = True
    while merged:
        merged = False
        for o, outer in enumerate(loops):
            for i, inner in enumerate(loops):
                if i != o and inner[0] == outer[0] and \
                        all(so == si * inner[1] for so, si in zip(outer[2], inner[2])):
                    outer[1] *= inner[1]
                    outer[2] = inner[2]
                    del loops[i]
                    merged = True
                    break
            if merged:
                break
    return (tuple(t for t, _, _ in loops), tuple(s for _, s, _ in loops),
            tuple(tuple(lp[2][k] for lp in loops) for k in range(len(strides))))


__all__ = ["TensorOperation", "TensorOperationConfig", "ConfigError", "DataType", "PrimType", "ExecType", "DimType",
           "ErrorType", "dtype", "float32", "float64", "bfloat16", "prim", "etype", "exec", "dim", "backend",
           "optimize"]
