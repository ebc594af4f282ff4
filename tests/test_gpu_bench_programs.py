"""The C++ harnesses (einsum_ir_amd/bin/bench_*: bench_binary, bench_unary,
bench_expression, bench_tree) on the GPU, on BASELINE configs 1, 2 and 4 and
on the reference's usage examples (reference src/bench_binary.cpp:219-230,
src/bench_unary.cpp:57-62, src/bench_expression.cpp:10-28,
src/bench_tree.cpp:8-20).  Each program drives the operator classes of
libeinsum_ir.so directly and checks its own result: a float64 host
evaluation (relative Frobenius error fp32 1e-5, fp64 1e-12, bf16 2e-3) or,
for permutations, bit equality.  A passing run exits 0 and prints its
correctness line."""
import os
import re
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "einsum_ir_amd", "bin")


def _run(prog, *args, timeout=180):
    print(f"running {prog} {' '.join(args)}", flush=True)
    sys.stdout.flush()
    res = subprocess.run([os.path.join(BIN, prog), *args], capture_output=True, text=True, timeout=timeout)
    assert res.returncode == 0, f"{prog} {args} exited {res.returncode}\n{res.stdout[-3000:]}\n{res.stderr[-3000:]}"
    return res.stdout


def _rel_error(out):
    return float(re.search(r"relative error:\s+(\S+)", out).group(1))


def test_bench_binary_config1():
    """abkl,cdkl->abcd, M=N=K=512 fp32, every output checked."""
    out = _run("bench_binary", "abkl,cdkl->abcd", "32,16,32,16,32,16", "FP32")
    assert "results are close" in out and "all output entries" in out
    assert _rel_error(out) <= 1e-5
    assert re.search(r"^CSV_DATA: einsum_ir,\"abkl,cdkl->abcd\"", out, re.M)
    assert "finished running bench_binary!" in out


@pytest.mark.parametrize("args", [
    ("abc,acdb->abd", "32,8,4,2", "FP32", "a,b,c,d"),                     # the reference's example
    ("[a,b,c],[a,c,d,b]->[a,b,d]", "32,8,4,2", "FP64"),
    ("zakm,zbkn->zabmn", "2,2,256,64,64,2", "BF16"),                      # config 3 kind, small
])
def test_bench_binary_examples(args):
    out = _run("bench_binary", *args)
    assert "results are close" in out


def test_bench_binary_config3_sampled():
    """BASELINE config 3 at full size: the host check restricts output dims."""
    out = _run("bench_binary", "zakm,zbkn->zabmn", "64,64,1024,64,64,8", "BF16")
    assert "results are close" in out and "output dims restricted to" in out
    assert _rel_error(out) <= 2e-3


def test_bench_unary_config2():
    """abcd->dbca on 64^4 fp32, bit-exact."""
    out = _run("bench_unary", "abcd->dbca", "64,64,64,64", "FP32")
    assert "results are equal (bit-exact, 16777216 entries)" in out
    assert re.search(r"^CSV_DATA: einsum_ir,\"abcd->dbca\",\"64,64,64,64\",FP32,134217728,", out, re.M)


@pytest.mark.parametrize("args", [("abcd->dbac", "32,32,32,32", "FP64"), ("abc->cab", "7,33,5", "BF16")])
def test_bench_unary_examples(args):
    assert "results are equal" in _run("bench_unary", *args)


def test_bench_expression_config4():
    """the 4-layer MLP chain bi,ih,hj,jk,ko->bo (b=4096,
    widths 2048), left to right -- in the path's standard form (operands
    removed, result appended) (0,1),(0,3),(0,2),(0,1); the host check samples
    rows of b."""
    out = _run("bench_expression", "bi,ih,hj,jk,ko->bo", "4096,2048,2048,2048,2048,2048",
               "(0,1),(0,3),(0,2),(0,1)", "FP32")
    assert "results are close" in out and "output dims restricted to b" in out
    assert _rel_error(out) <= 1e-5
    flops = int(re.search(r"#flops:\s+(\d+)", out).group(1))
    assert flops == 4 * (2 * 4096 * 2048 * 2048 - 4096 * 2048)


EXAMPLE = ("iae,bf,dcba,cg,dh->hgfei", "32,8,4,2,16,64,8,8,8", "(1,2),(2,3),(0,1),(0,1)")


@pytest.mark.parametrize("dtype,store_lock", [("FP32", "0"), ("FP64", "1"), ("CPX_FP32", "0"), ("CPX_FP64", "1")])
def test_bench_expression_examples(dtype, store_lock):
    out = _run("bench_expression", *EXAMPLE, dtype, store_lock)
    assert "results are close" in out


def test_bench_expression_standard_and_numeric_names():
    for expr in ("[i,a,e],[b,f],[d,c,b,a],[c,g],[d,h]->[h,g,f,e,i]",
                 "[8,0,4],[1,5],[3,2,1,0],[2,6],[3,7]->[7,6,5,4,8]"):
        assert "results are close" in _run("bench_expression", expr, *EXAMPLE[1:])


def test_print_tree_round_trip():
    """print_tree 1 writes the compiled tree in the exchange format; bench_tree
    evaluates that string with the same sizes (ids are the sorted names'
    positions) and matches its own host evaluation.  Modes 2-4 print the same
    tree with names / drawn."""
    out = _run("bench_expression", *EXAMPLE, "FP32", "0", "1")
    lines = out.splitlines()
    tree = lines[lines.index("*** benchmarking einsum_ir ***") + 1]
    assert tree.endswith("->[7,6,5,4,8]") and tree.count("->") >= 4, tree
    assert "results are close" in _run("bench_tree", tree, EXAMPLE[1], "FP32")
    named = _run("bench_expression", *EXAMPLE, "FP32", "0", "2").splitlines()
    named_tree = named[named.index("*** benchmarking einsum_ir ***") + 1]
    assert named_tree.endswith("->[h,g,f,e,i]") and not re.search(r"\d", named_tree), named_tree
    drawn = _run("bench_expression", *EXAMPLE, "FP32", "0", "4").splitlines()
    first = drawn.index("*** benchmarking einsum_ir ***") + 1
    assert drawn[first].split() == ["h", "g", "f", "e", "i"]       # the root's line
    assert any(set(line.split()) >= {"d", "c", "b", "a"} for line in drawn[first:first + 8])


def test_print_tree_one_child_root():
    """A complex BATCH_INNER tree ends in a one-child node (the conversion of
    the complex-outermost result); the exchange format writes such a node as
    its own ids only, without its subtree, as the reference does
    (src/frontend/EinsumExpression.cpp:504-563).  The real tree of the same
    expression keeps its full nesting."""
    args = ("ab,bc->ac", "3,4,5", "(0,1)")
    real = _run("bench_expression", *args, "FP32", "0", "1").splitlines()
    real_tree = real[real.index("*** benchmarking einsum_ir ***") + 1]
    assert real_tree.startswith("[") and "],[" in real_tree and real_tree.endswith("->[0,2]"), real_tree
    cpx = _run("bench_expression", *args, "CPX_FP32", "0", "1").splitlines()
    cpx_tree = cpx[cpx.index("*** benchmarking einsum_ir ***") + 1]
    assert re.fullmatch(r"\d+(,\d+)*", cpx_tree) and "->" not in cpx_tree, cpx_tree
    assert cpx_tree.split(",")[:2] == ["0", "2"], cpx_tree


@pytest.mark.parametrize("args", [
    ("[[3,0]->[0,3]],[[3,2,4],[1,4,2]->[1,2,3]]->[0,1,2]", "2,3,4,5,6", "FP32"),   # the reference's example
    ("[[3,0]->[0,3]],[[3,2,4],[1,4,2]->[1,2,3]]->[0,1,2]", "20,30,40,50,60", "FP64"),
])
def test_bench_tree_examples(args):
    out = _run("bench_tree", *args)
    assert "results are close" in out
    assert re.search(r"^CSV_DATA: einsum_ir,", out, re.M)
