"""GPU parity on the reference's sample workloads (tests/golden/einsum_samples.json,
shape data of reference samples/tccg/*.cfg and samples/einsum_benchmark/*.cfg).

* TCCG: the 59 binary contractions of the TCCG suite, which the reference runs
  through bench_expression with path (0,1), fp32, at their full sizes.
* einsum_benchmark: the real-world tensor networks (language-model and MERA
  networks, the synthetic tree), as expressions with the recorded path and as
  the recorded einsum trees (bench_tree format).

Checker: torch.einsum in float64 on the GPU, pair by pair along the same path
or tree (the library routine the oracle is pinned to; these sizes are far
beyond what the CPU oracle finishes in seconds).  Inputs are N(0,1), each
tensor scaled by prod(size of its contracted dims)^-1/4 so that long networks
stay in fp32 range.  Bar: relative Frobenius error <= 1e-5 (fp32).

The two language-model networks (2.8 and 7.1 TFLOP) run here at two sets of
reduced mode sizes (same expression, path and tree); at full size they are
benchmarked by bench.py.
"""
import json
import os

import pytest

import einsum_ir_amd as eir
from einsum_ir_amd import harness, host
from tests.helpers import TOL_FP32

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
with open(os.path.join(ROOT, "tests", "golden", "einsum_samples.json")) as _f:
    SAMPLES = json.load(_f)

# reduced mode sizes of the language-model networks: "s" (~10 MFLOP) and "m"
# (2-8 GFLOP, odd sizes 5 for ragged tiles)
REDUCE = {"s": {16: 4, 11: 3, 7: 3, 128: 8}, "m": {16: 8, 11: 5, 7: 5, 128: 16}}


def _rel(torch, ref, got):
    ref = ref.double()
    got = got.double()
    return float(torch.linalg.vector_norm(ref - got) / torch.linalg.vector_norm(ref))


def _run_expression(torch, expr, sizes_arg, path_arg, seed):
    ins, out = harness._tensors(expr)
    sizes = harness._sizes(expr, sizes_arg)
    path = harness._parse_path(path_arg)
    data = harness.scaled_randn(torch, ins, out, sizes, seed, torch.float32)
    dout = torch.zeros([sizes[d] for d in out], device="cuda", dtype=torch.float32)
    e = host.Expression(expr, sizes, path, data + [dout], dtype=eir.FP32)
    e.eval()
    ref = harness.torch_path_eval(torch, ins, out, sizes, path, [d.double() for d in data])
    err = _rel(torch, ref, dout)
    n = e.num_ops()
    e.close()
    return err, n


@pytest.mark.parametrize("case", SAMPLES["tccg"], ids=lambda c: c["expr"])
def test_tccg_fp32(torch_cuda, case):
    err, n = _run_expression(torch_cuda, case["expr"], case["sizes"], case["path"],
                             seed=sum(map(ord, case["expr"])))
    print(f"{case['expr']} sizes={case['sizes']} flops={n} rel_err={err:.3e}", flush=True)
    assert n > 0
    assert err <= TOL_FP32


def _sample_sizes(name, key, red):
    s = SAMPLES["einsum_benchmark"][name][key]
    if not red:
        return s
    return ",".join(str(REDUCE[red].get(int(x), int(x))) for x in s.split(","))


def _cases(key):
    out = []
    for name, c in SAMPLES["einsum_benchmark"].items():
        if key in c:
            out += [(name, r) for r in REDUCE] if name.startswith("lm_") else [(name, "")]
    return out


@pytest.mark.parametrize("name,red", _cases("expr"))
def test_einsum_benchmark_expression_fp32(torch_cuda, name, red):
    c = SAMPLES["einsum_benchmark"][name]
    sizes = _sample_sizes(name, "sizes", red)
    err, n = _run_expression(torch_cuda, c["expr"], sizes, c["path"], seed=11)
    print(f"{name} {red} flops={n} rel_err={err:.3e}", flush=True)
    assert err <= TOL_FP32


@pytest.mark.parametrize("name,red", _cases("tree"))
def test_einsum_benchmark_tree_fp32(torch_cuda, name, red):
    torch = torch_cuda
    c = SAMPLES["einsum_benchmark"][name]
    sizes = [int(x) for x in _sample_sizes(name, "tree_sizes", red).split(",")]
    nodes = harness._parse_tree(c["tree"])
    leaves = [dims for dims, kids in nodes if not kids]
    root_dims = nodes[-1][0]
    sz = dict(enumerate(sizes))
    data = iter(harness.scaled_randn(torch, leaves, root_dims, sz, 12, torch.float32))
    tensors = [next(data) if not kids else None for dims, kids in nodes]
    root = torch.zeros([sizes[d] for d in root_dims], device="cuda", dtype=torch.float32)
    tensors[-1] = root
    tr = host.Tree(c["tree"], sizes, tensors, dtype=eir.FP32)
    tr.eval()
    ref = harness.torch_tree_eval(torch, nodes, tensors[:-1] + [None], torch.float64)[-1]
    err = _rel(torch, ref, root)
    print(f"{name} {red} tree flops={tr.num_ops()} rel_err={err:.3e}", flush=True)
    tr.close()
    assert err <= TOL_FP32
