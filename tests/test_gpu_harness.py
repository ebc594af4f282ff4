"""The reference's command-line harnesses on the HIP backend
(einsum_ir_amd.harness: bench_binary, bench_unary, bench_expression,
bench_tree with the reference's argument formats, reference
src/bench_*.cpp).  Each run compares its result with torch (allclose with
the reference harnesses' rtol 1e-3 / atol 1e-4, bit equality for the
permutation) and returns non-zero otherwise; the tests check the return code
and the CSV_DATA report."""
import pytest

from einsum_ir_amd import harness

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("argv", [
    ["binary", "abkl,cdkl->abcd", "32,16,32,16,32,16", "FP32"],
    ["binary", "abc,acdb->abd", "32,8,4,2", "FP64", "a,b,c,d"],          # the reference's usage example
    ["binary", "[x,y],[y,z]->[x,z]", "64,48,40", "BF16"],                 # standard format, bf16
    ["unary", "abcd->dbca", "16,24,8,12", "FP32"],
    ["unary", "abcd->dbac", "32,32,32,32", "FP64"],                       # the reference's usage example
    ["expression", "iae,bf,dcba,cg,dh->hgfei", "32,8,4,2,16,64,8,8,8", "(1,2),(2,3),(0,1),(0,1)"],
    ["expression", "iae,bf,dcba,cg,dh->hgfei", "32,8,4,2,16,64,8,8,8", "(1,2),(2,3),(0,1),(0,1)", "FP64", "1"],
    ["expression", "km,nk->nm", "4,2,3", "(0,1)", "CPX_FP32"],
    ["tree", "[[3,0]->[0,3]],[[3,2,4],[1,4,2]->[1,2,3]]->[0,1,2]", "2,3,4,5,6", "FP32"],
])
def test_harness(torch_cuda, capsys, argv):
    rc = harness.main(argv)
    out = capsys.readouterr().out
    assert rc == 0, out
    assert "CSV_DATA: einsum_ir," in out
